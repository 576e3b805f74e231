"""tenzo_hip_attn_int8_decode_noalloc (the entry point that allocates nothing:
its chunk partials live in a fixed device array) against
tenzo_hip_attn_int8_decode on the same inputs, through the C ABI: output,
rotated q/k and the appended cache rows bit-exact (the same kernels, only the
partials' address differs). Two calls in a row, the second smaller (the array
keeps the first call's contents), then a call too large for the array, which
must be refused without touching the outputs."""
import ctypes

import numpy as np
import pytest

from tenzo_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch
    assert torch.cuda.is_available(), "GPU test needs a visible GPU"
    from tenzo_amd import _lib, ops
    return torch, _lib.load(), ops


def _inputs(torch, rng, B, Hq, Hkv, max_seq, pos, zeros=False):
    if zeros:
        kc = np.zeros((B, Hkv, max_seq, 128), np.int8)
        ks = np.full((B, Hkv, max_seq), 0.02, np.float16)
        q = np.zeros((B, Hq * 128), np.float32)
        k = np.zeros((B, Hkv * 128), np.float32)
        return q, k, k, kc, kc, ks, ks
    kc = rng.integers(-127, 128, size=(B, Hkv, max_seq, 128), dtype=np.int8)
    vc = rng.integers(-127, 128, size=(B, Hkv, max_seq, 128), dtype=np.int8)
    ks = synth.f16_round(rng.uniform(0.01, 0.04, size=(B, Hkv, max_seq))).astype(np.float16)
    vs = synth.f16_round(rng.uniform(0.01, 0.04, size=(B, Hkv, max_seq))).astype(np.float16)
    q = rng.standard_normal((B, Hq * 128)).astype(np.float32)
    k = rng.standard_normal((B, Hkv * 128)).astype(np.float32)
    v = rng.standard_normal((B, Hkv * 128)).astype(np.float32)
    return q, k, v, kc, vc, ks, vs


def _run(torch, L, ops, name, host, Hq, pos, theta=500000.0):
    q, k, v, kc, vc, ks, vs = host
    B, Hkv, max_seq, _ = kc.shape
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    tq, tk, tv, tkc, tvc, tks, tvs = (dev(a) for a in (q, k, v, kc, vc, ks, vs))
    cs = ops.rope_table(theta, pos, 1)[0].cuda()
    out = torch.full((B, Hq * 128), -7.0, dtype=torch.float32, device="cuda")
    q_rot = torch.empty_like(out)
    k_rot = torch.empty((B, Hkv * 128), dtype=torch.float32, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    torch.cuda.synchronize()
    rc = getattr(L, name)(P(tq), P(tk), P(tv), P(tkc), P(tvc), P(tks), P(tvs), P(cs), B, Hq, Hkv,
                          max_seq, pos, P(out), P(q_rot), P(k_rot),
                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return rc, [t.cpu().numpy() for t in (out, q_rot, k_rot, tkc, tvc, tks, tvs)]


@pytest.mark.parametrize("B,Hq,Hkv,ctx", [(4, 20, 5, 8192), (1, 20, 5, 1500)])
def test_noalloc_matches_attn_int8_decode(env, B, Hq, Hkv, ctx):
    """Run in order: the larger call first, then the smaller one over the
    array the first left behind."""
    torch, L, ops = env
    print(f"noalloc B={B} Hq={Hq} Hkv={Hkv} ctx={ctx}", flush=True)
    rng = np.random.default_rng(ctx + B)
    pos = ctx - 1
    host = _inputs(torch, rng, B, Hq, Hkv, ctx + 8, pos)
    rc0, ref = _run(torch, L, ops, "tenzo_hip_attn_int8_decode", host, Hq, pos)
    assert rc0 == 0
    for rep in range(2):
        rc1, got = _run(torch, L, ops, "tenzo_hip_attn_int8_decode_noalloc", host, Hq, pos)
        assert rc1 == 0, L.tenzo_hip_last_error()
        for g, r in zip(got, ref):
            np.testing.assert_array_equal(g, r)


def test_noalloc_refuses_oversized(env):
    """B 16 at context 32768: 128 chunks x 16 x 20 query heads x 520 bytes =
    21 MB of partials > 8 MiB: refused before any launch."""
    torch, L, ops = env
    B, Hq, Hkv, ctx = 16, 20, 5, 32768
    rng = np.random.default_rng(3)
    host = _inputs(torch, rng, B, Hq, Hkv, ctx, ctx - 1, zeros=True)
    rc, got = _run(torch, L, ops, "tenzo_hip_attn_int8_decode_noalloc", host, Hq, ctx - 1)
    assert rc == -1  # TENZO_ERROR_INVALID_ARGUMENT
    assert b"exceed" in L.tenzo_hip_last_error()
    assert (got[0] == -7.0).all()  # nothing was written
