"""tenzo_load_model on the GPU: the raw-layout repack and the LM-head
quantization against the oracle (bit-exact), and an engine loaded from
weights.bin + model.mlir against an engine given what the compiled
reference's own loader made of the same files (bit-exact). (The decode step
itself is compared with the reference elsewhere; with fp16 KV scales it
departs from the reference's fp32 scales by more than rounding once several
kv heads feed one activation quantizer, see the engine tests.)"""
import ctypes

import numpy as np
import pytest

import oracle
from tests import model_files

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU test needs a visible GPU"
    from tenzo_amd import _lib
    _lib.load()
    return torch


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("N,K", [(64, 64), (128, 130), (192, 1000), (2560, 2560), (640, 2560),
                                 (2560, 6912), (6912, 2560)])
def test_repack_raw_equals_repack_of_packed(torch_dev, N, K):
    """Device layout from the loader's raw bytes = device layout of the TL1
    blocks pack_ternary_weights_raw makes of them (oracle packer, itself
    pinned against the reference's)."""
    from tenzo_amd import _lib, ops
    torch = torch_dev
    rng = np.random.default_rng(N + K)
    _, raw = model_files.raw_ternary(N, K, rng)
    tl1 = oracle.tl1_pack_raw(raw, N, K)
    want = ops.tl1_repack(torch.from_numpy(tl1).cuda(), N, K)
    got = torch.empty_like(want)
    _lib.check(_lib.load().tenzo_hip_tl1_repack_raw(_ptr(torch.from_numpy(raw).cuda()),
                                                    _ptr(got), N, K, None), "repack_raw")
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_quant_rows_i8_matches_oracle(torch_dev):
    from tenzo_amd import _lib
    torch = torch_dev
    rng = np.random.default_rng(5)
    E = (rng.standard_normal((333, 2560)) * rng.uniform(0.001, 1.0, (333, 1))).astype(np.float32)
    E[3] = 0.0
    E[4, 7] = 1e30
    dE = torch.from_numpy(E).cuda()
    codes = torch.empty((333, 2560), dtype=torch.int8, device="cuda")
    scales = torch.empty(333, dtype=torch.float32, device="cuda")
    _lib.check(_lib.load().tenzo_hip_quant_rows_i8(_ptr(dE), 333, 2560, _ptr(codes),
                                                   _ptr(scales), None), "quant_rows_i8")
    oc, os_ = oracle.quant_rows_i8(E)
    assert np.array_equal(codes.cpu().numpy(), oc)
    assert np.array_equal(scales.cpu().numpy(), os_)


@pytest.mark.skipif(not oracle.ref_available(), reason="compiled reference not built")
@pytest.mark.parametrize("variant", ["all", "views5", "truncated"])
def test_engine_load_model_equals_reference_loaders_model(torch_dev, tmp_path, variant):
    """An engine loaded from weights.bin + model.mlir equals, bit for bit over
    several greedy steps (tokens, logits, hidden state, KV cache), an engine
    given the arrays the compiled reference's own loader produced from the
    same files (TL1 blocks, scales, norms, int8 LM head, final norm) through
    tenzo_set_layer_weights / tenzo_set_lm_head_i8 / tenzo_set_final_norm."""
    from tenzo_amd import engine as eng_mod, synth
    H, Hq, Hkv, F, L, V = 2560, 20, 5, 512, 2, 320
    kw = {"views": 5} if variant == "views5" else {}
    if variant == "truncated":
        kw["truncate"] = V * H * 4 + 5_000_000
    wpath, mpath, _ = model_files.write(str(tmp_path), H=H, Hq=Hq, Hkv=Hkv, F=F, L=L, V=V,
                                        seed=13, **kw)
    print(f"load_model {variant}", flush=True)
    R = oracle.ref()
    re_ = R.ref_engine_create(H, Hq, Hkv, L, F, V, 16)
    cfg = synth.DecodeConfig(hidden=H, n_q_heads=Hq, n_kv_heads=Hkv, n_layers=L, ffn=F,
                             vocab=V, max_seq=16, theta=10000.0)
    keep = []
    try:
        assert R.ref_engine_load(re_, wpath.encode(), mpath.encode()) == 0
        with eng_mod.Engine(cfg) as a, eng_mod.Engine(cfg) as b:
            a.load_model(wpath, mpath)
            for l in range(L):
                lw = eng_mod.LayerWeights()
                for which, f in enumerate(["q", "k", "v", "out", "gate", "up", "down"]):
                    n = R.ref_engine_layer_data(re_, l, which, None, None)
                    buf = np.empty(n, np.int8)
                    sc = ctypes.c_float()
                    R.ref_engine_layer_data(re_, l, which, buf.ctypes.data, ctypes.byref(sc))
                    keep.append(buf)
                    setattr(lw, f + "_w", buf.ctypes.data)
                    setattr(lw, f + "_scale", sc.value)
                for which, f in enumerate(["in_norm", "attn_sub_norm", "post_norm",
                                           "ffn_sub_norm"], 7):
                    n = R.ref_engine_layer_data(re_, l, which, None, None)
                    buf = np.empty(n, np.float32)
                    R.ref_engine_layer_data(re_, l, which, buf.ctypes.data, None)
                    keep.append(buf)
                    setattr(lw, f, buf.ctypes.data)
                b._check(b.L.tenzo_set_layer_weights(b.h, l, ctypes.byref(lw)), "set_layer")
            codes = np.empty((V, H), np.int8)
            hs = np.empty(V, np.float32)
            fin = np.empty(H, np.float32)
            R.ref_engine_head_data(re_, codes.ctypes.data, hs.ctypes.data, fin.ctypes.data)
            b._check(b.L.tenzo_set_lm_head_i8(b.h, codes.ctypes.data, hs.ctypes.data, V, H),
                     "head")
            b._check(b.L.tenzo_set_final_norm(b.h, fin.ctypes.data), "final_norm")
            ta = tb = 17
            for _ in range(4):
                ta, tb = a.step(ta), b.step(tb)
                assert ta == tb
                np.testing.assert_array_equal(a.logits(), b.logits())
                np.testing.assert_array_equal(a.buffer("x"), b.buffer("x"))
            for u, v in zip(a.get_kv(4), b.get_kv(4)):
                np.testing.assert_array_equal(u, v)
    finally:
        R.ref_engine_destroy(re_)


def test_engine_load_model_errors(torch_dev, tmp_path):
    from tenzo_amd import engine as eng_mod, synth
    cfg = synth.DecodeConfig(hidden=512, n_q_heads=4, n_kv_heads=1, n_layers=1, ffn=512,
                             vocab=256, max_seq=16, theta=10000.0)
    wpath, mpath, _ = model_files.write(str(tmp_path), H=512, Hq=4, Hkv=1, F=512, L=1, V=256,
                                        seed=1, truncate=1000)
    with eng_mod.Engine(cfg) as e:
        with pytest.raises(RuntimeError, match="embedding"):
            e.load_model(wpath, mpath)
        with pytest.raises(RuntimeError, match="cannot open"):
            e.load_model(str(tmp_path / "missing.bin"), mpath)
