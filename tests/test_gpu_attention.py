"""INT8 KV decode attention on the GPU against the CPU oracle (same RoPE table,
fp16 cache scales) and the compiled-reference goldens. Appended KV codes and
rotated q/k are bit-exact; attention outputs are within 1e-3 relative."""
import os

import numpy as np
import pytest

import oracle
from tenzo_amd import synth

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
RTOL = 1e-3


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU test needs a visible GPU"
    from tenzo_amd import _lib
    _lib.load()
    return torch


def make_cache(rng, B, Hkv, max_seq, ctx):
    kc = np.zeros((B, Hkv, max_seq, 128), np.int8)
    vc = np.zeros_like(kc)
    ks = np.zeros((B, Hkv, max_seq), np.float32)
    vs = np.zeros_like(ks)
    if ctx and B * ctx <= 8192:
        for c, s in ((kc, ks), (vc, vs)):
            codes, sc = synth.kv_quantize(rng.standard_normal((B, Hkv, ctx, 128)).astype(np.float32))
            c[:, :, :ctx] = codes
            s[:, :, :ctx] = synth.f16_round(sc)
    elif ctx:  # long contexts: random codes and scales of the same ranges (faster to make)
        for c, s in ((kc, ks), (vc, vs)):
            c[:, :, :ctx] = rng.integers(-127, 128, size=(B, Hkv, ctx, 128), dtype=np.int8)
            s[:, :, :ctx] = synth.f16_round(rng.uniform(0.01, 0.04, size=(B, Hkv, ctx)))
    return kc, vc, ks, vs


def run_gpu(torch, q, k, v, kc, vc, ks, vs, pos, theta):
    from tenzo_amd import ops
    B, Hkv, max_seq, _ = kc.shape
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    tkc, tvc = dev(kc), dev(vc)
    tks = dev(ks.astype(np.float16))
    tvs = dev(vs.astype(np.float16))
    cs = ops.rope_table(theta, pos, 1)[0].cuda()
    out, q_rot, k_rot = ops.attn_int8_decode(dev(q), dev(k), dev(v), tkc, tvc, tks, tvs, cs, pos,
                                             want_rot=True)
    torch.cuda.synchronize()
    return (out.cpu().numpy(), q_rot.cpu().numpy(), k_rot.cpu().numpy(), tkc.cpu().numpy(),
            tvc.cpu().numpy(), tks.cpu().numpy().astype(np.float32),
            tvs.cpu().numpy().astype(np.float32))


def run_oracle(q, k, v, kc, vc, ks, vs, Hq, pos, theta):
    B, Hkv, max_seq, _ = kc.shape
    cs = oracle.rope_table(theta, pos)
    outs, qrs, krs = [], [], []
    kc, vc, ks, vs = kc.copy(), vc.copy(), ks.copy(), vs.copy()
    for b in range(B):
        o, qr, kr = oracle.attention_step(q[b], k[b], v[b], kc[b], vc[b], ks[b], vs[b], Hq, Hkv,
                                          max_seq, pos, cs, f16_scales=True)
        outs.append(o)
        qrs.append(qr)
        krs.append(kr)
    return np.stack(outs), np.stack(qrs), np.stack(krs), kc, vc, ks, vs


def check(gpu, ref, pos):
    out, q_rot, k_rot, kc, vc, ks, vs = gpu
    o_ref, q_ref, k_ref, kc_r, vc_r, ks_r, vs_r = ref
    np.testing.assert_array_equal(q_rot, q_ref)
    np.testing.assert_array_equal(k_rot, k_ref)
    np.testing.assert_array_equal(kc[:, :, pos], kc_r[:, :, pos])
    np.testing.assert_array_equal(vc[:, :, pos], vc_r[:, :, pos])
    np.testing.assert_array_equal(ks[:, :, pos], ks_r[:, :, pos])
    np.testing.assert_array_equal(vs[:, :, pos], vs_r[:, :, pos])
    np.testing.assert_array_equal(kc[:, :, :pos], kc_r[:, :, :pos])
    np.testing.assert_allclose(out, o_ref, rtol=RTOL, atol=RTOL * 1e-2 * np.abs(o_ref).max())
    rel = np.abs(out - o_ref).max() / np.abs(o_ref).max()
    print(f"  max rel err {rel:.2e}", flush=True)
    assert rel < RTOL


@pytest.mark.parametrize("B,Hq,Hkv,ctx", [(1, 20, 5, 1), (1, 20, 5, 37), (1, 20, 5, 1024),
                                          (1, 20, 5, 4096), (16, 20, 5, 1024), (1, 8, 1, 300),
                                          (2, 4, 2, 700), (1, 8, 1, 8192), (1, 5, 5, 100),
                                          (1, 20, 5, 8192), (16, 20, 5, 8192)])
def test_attention_matches_oracle(torch_dev, B, Hq, Hkv, ctx):
    print(f"attention B={B} Hq={Hq} Hkv={Hkv} ctx={ctx}", flush=True)
    rng = np.random.default_rng(B * 1000 + ctx)
    max_seq = ctx + 3
    pos = ctx - 1  # the appended token is the ctx-th
    kc, vc, ks, vs = make_cache(rng, B, Hkv, max_seq, pos)
    q = rng.standard_normal((B, Hq * 128)).astype(np.float16).astype(np.float32)
    k = rng.standard_normal((B, Hkv * 128)).astype(np.float32)
    v = rng.standard_normal((B, Hkv * 128)).astype(np.float32)
    for theta in (10000.0, 500000.0):
        gpu = run_gpu(torch_dev, q, k, v, kc, vc, ks, vs, pos, theta)
        ref = run_oracle(q, k, v, kc, vc, ks, vs, Hq, pos, theta)
        check(gpu, ref, pos)


def test_attention_long_context_32k(torch_dev):
    """Config-5 layout at 32k context, batch 1 and 16, every sequence checked
    against the oracle."""
    rng = np.random.default_rng(77)
    for B, ctx in ((1, 32768), (16, 32768)):
        print(f"attention 32k B={B}", flush=True)
        Hq, Hkv = 20, 5
        pos = ctx - 1
        kc, vc, ks, vs = make_cache(rng, B, Hkv, ctx, pos)
        q = rng.standard_normal((B, Hq * 128)).astype(np.float16).astype(np.float32)
        k = rng.standard_normal((B, Hkv * 128)).astype(np.float32)
        v = rng.standard_normal((B, Hkv * 128)).astype(np.float32)
        gpu = run_gpu(torch_dev, q, k, v, kc, vc, ks, vs, pos, 500000.0)
        ref = run_oracle(q, k, v, kc, vc, ks, vs, Hq, pos, 500000.0)
        check(gpu, ref, pos)


def test_attention_single_token_is_dequantized_v(torch_dev):
    rng = np.random.default_rng(5)
    B, Hq, Hkv = 1, 20, 5
    kc, vc, ks, vs = make_cache(rng, B, Hkv, 4, 0)
    q = rng.standard_normal((B, Hq * 128)).astype(np.float32)
    k = rng.standard_normal((B, Hkv * 128)).astype(np.float32)
    v = rng.standard_normal((B, Hkv * 128)).astype(np.float32)
    out, _, _, _, vc_g, _, vs_g = run_gpu(torch_dev, q, k, v, kc, vc, ks, vs, 0, 10000.0)
    for qh in range(Hq):
        h = qh // 4
        np.testing.assert_allclose(out[0, qh * 128:(qh + 1) * 128],
                                   vc_g[0, h, 0].astype(np.float32) * vs_g[0, h, 0], rtol=1e-6)


def test_attention_matches_reference_goldens(torch_dev):
    z = np.load(os.path.join(GOLD, "attention.npz"))
    for tag in "abc":
        Hq, Hkv, max_seq, pos = (int(x) for x in z[f"{tag}_dims"])
        print(f"golden {tag}: Hq={Hq} Hkv={Hkv} pos={pos}", flush=True)
        gpu = run_gpu(torch_dev, z[f"{tag}_in_q"][None], z[f"{tag}_in_k"][None],
                      z[f"{tag}_in_v"][None], z[f"{tag}_in_kc"][None], z[f"{tag}_in_vc"][None],
                      z[f"{tag}_in_ks"][None], z[f"{tag}_in_vs"][None], pos, 10000.0)
        out, q_rot, k_rot, kc, vc, ks, vs = (g[0] for g in gpu)
        np.testing.assert_array_equal(q_rot, z[f"{tag}_q_rot"])
        np.testing.assert_array_equal(k_rot, z[f"{tag}_k_rot"])
        np.testing.assert_array_equal(kc[:, pos], z[f"{tag}_kc"][:, pos])
        np.testing.assert_array_equal(vc[:, pos], z[f"{tag}_vc"][:, pos])
        np.testing.assert_array_equal(ks[:, pos], synth.f16_round(z[f"{tag}_ks"][:, pos]))
        ref = z[f"{tag}_out"]
        assert np.abs(out - ref).max() / np.abs(ref).max() < RTOL
