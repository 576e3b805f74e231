"""GGUF Q4_0 (fp16 / fp32 / Q8_0 activations), GGUF Q8_0, GPTQ and AWQ GEMVs on
the GPU against the CPU oracle (bit-exact with the compiled reference for the
GGUF formats) and the compiled-reference goldens, at the benchmark shapes (Q4_0
and Q8_0 11008x4096; GPTQ/AWQ K=4096 N=14336 group 128, batch 1 and 8).

These are fp32 reductions in another order than the reference's, so each
output is held to the forward-error bound of fp32 summation, which no order
can exceed: with the terms t_k = a_k w_k (w dequantized exactly),
|y - sum t| <= gamma_n sum |t_k| for any order with n roundings on the
longest path (gamma_n = n u / (1 - n u), u = 2^-24), so two orders differ by
at most 2 gamma_n sum |t_k|, taken with n = K + 8. The run prints how much of
that bound is used, and the north star's 1e-3 (relative to the largest |y|
of the call) is checked as well."""
import os

import numpy as np
import pytest

import oracle
from tenzo_amd import formats, synth

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


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


U = 2.0 ** -24


def close(y, ref, a=None, W=None):
    """y vs ref (both [..., N]); with the activations a [.., K] and the
    dequantized weights W [N][K], also the summation bound above."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(y - ref)
    rel = err.max() / np.abs(ref).max()
    msg = f"  max err / max|y| = {rel:.2e}"
    if W is not None:
        K = W.shape[1]
        n = K + 8
        gamma = n * U / (1 - n * U)
        mag = np.abs(np.asarray(a, np.float64)) @ np.abs(W).T  # sum_k |a_k w_nk|
        tol = 2 * gamma * mag
        used = (err / np.maximum(tol, 1e-300)).max()
        msg += f", of the summation bound: {used:.2e}"
        assert (err <= tol).all(), msg
    print(msg, flush=True)
    assert rel < RTOL


def q4_dense(q, d):
    return (q.astype(np.float64) - 8) * np.repeat(d.astype(np.float64), 32, axis=1)


def make_q4(rng, N, K, dense=False):
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    d = np.abs(rng.normal(0, 0.01, size=(N, K // 32))).astype(np.float16)
    w = formats.q4_0_pack(q, d)
    return (w, q4_dense(q, d)) if dense else w


@pytest.mark.parametrize("N,K", [(64, 32), (100, 256), (11008, 4096), (257, 4128), (72, 2304),
                                 (40, 8192)])
def test_q4_0_fp16_and_fp32_activations(torch_dev, N, K):
    from tenzo_amd import ops
    torch = torch_dev
    print(f"q4_0 N={N} K={K}", flush=True)
    rng = np.random.default_rng(N + K)
    w, W = make_q4(rng, N, K, dense=True)
    a16 = rng.standard_normal(K).astype(np.float16)
    a = a16.astype(np.float32)
    ref = oracle.q4_0(a, w, K, N)
    y = ops.gemv_q4_0(dev(torch, a16), dev(torch, w), K, N).cpu().numpy()[0]
    close(y, ref, a, W)
    y32 = ops.gemv_q4_0(dev(torch, a), dev(torch, w), K, N).cpu().numpy()[0]
    close(y32, ref, a, W)


@pytest.mark.parametrize("N,K,B", [(64, 32, 1), (100, 288, 2), (11008, 4096, 1),
                                   (11008, 4096, 8), (257, 4128, 1), (72, 2304, 2),
                                   (40, 8192, 1), (24, 16384, 1), (1003, 4096, 1),
                                   (5, 2048, 3)])
def test_q8_0_weights(torch_dev, N, K, B):
    """compute_linear_gguf_q8_0 (TenzoEngine.cpp:1078-1114). K = 288 and 4128
    leave rows that are not 16-byte aligned or a partial group of 8 blocks
    (the halfword path); K = 2048, 2304 and 4096 stage 8 rows at a time
    through LDS (N = 1003 and 5 end in a partial block of rows), 8192 and
    16384 take the 16-byte loads per lane."""
    from tenzo_amd import ops
    torch = torch_dev
    print(f"q8_0 N={N} K={K} B={B}", flush=True)
    rng = np.random.default_rng(3 * N + K + B)
    q = rng.integers(-127, 128, size=(N, K)).astype(np.int8)
    d = np.abs(rng.normal(0, 0.01, size=(N, K // 32))).astype(np.float16)
    w = formats.q8_0_pack(q, d)
    W = q.astype(np.float64) * np.repeat(d.astype(np.float64), 32, axis=1)
    a16 = rng.standard_normal((B, K)).astype(np.float16)
    a = a16.astype(np.float32)
    ref = np.stack([oracle.q8_0(a[b], w, K, N) for b in range(B)])
    y = ops.gemv_q8_0(dev(torch, a16), dev(torch, w), K, N).cpu().numpy()
    close(y, ref, a, W)
    y32 = ops.gemv_q8_0(dev(torch, a), dev(torch, w), K, N).cpu().numpy()
    np.testing.assert_array_equal(y32, y)  # the same fp32 activations either way


@pytest.mark.parametrize("N,K", [(64, 32), (11008, 4096), (100, 2304), (257, 8192), (33, 288)])
def test_q4_0_q8_0_activations(torch_dev, N, K):
    from tenzo_amd import ops
    torch = torch_dev
    rng = np.random.default_rng(7 + N)
    w = make_q4(rng, N, K)
    x = rng.standard_normal(K).astype(np.float16).astype(np.float32)
    qa = oracle.quantize_q8_0(x)
    ref = oracle.q4_0_q8act(qa, w, K, N)
    y = ops.gemv_q4_0_q8_0(dev(torch, qa), dev(torch, w), K, N).cpu().numpy()[0]
    close(y, ref)


def test_quant_gemv_reference_goldens(torch_dev):
    from tenzo_amd import ops
    torch = torch_dev
    z = np.load(os.path.join(GOLD, "quant_gemv.npz"))
    K, N, G = (int(v) for v in z["dims"])
    a = dev(torch, z["a"])
    close(ops.gemv_q4_0(a, dev(torch, z["q4_w"]), K, N).cpu().numpy()[0], z["q4_y"])
    close(ops.gemv_q8_0(a, dev(torch, z["q8_w"]), K, N).cpu().numpy()[0], z["q8_y"])
    sc = dev(torch, z["scales"])
    for kind, fn in (("gptq", ops.gemv_gptq), ("awq", ops.gemv_awq)):
        y = fn(a, dev(torch, z[f"{kind}_qweight"]), sc, dev(torch, z[f"{kind}_qzeros"]), K, N,
               G).cpu().numpy()[0]
        close(y, z[f"{kind}_y"])


@pytest.mark.parametrize("kind", ["gptq", "awq"])
@pytest.mark.parametrize("B", [1, 8])
def test_gptq_awq_benchmark_shape(torch_dev, kind, B):
    from tenzo_amd import ops
    torch = torch_dev
    print(f"{kind} B={B}", flush=True)
    K, N, G = 4096, 14336, 128
    rng = np.random.default_rng(11 + B)
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    zeros = rng.integers(0, 16, size=(K // G, N), dtype=np.uint8)
    scales16 = np.abs(rng.normal(0, 0.01, size=(K // G, N))).astype(np.float16)
    pack = formats.gptq_pack if kind == "gptq" else formats.awq_pack
    qw, qz = pack(q, zeros)
    a = rng.standard_normal((B, K)).astype(np.float16)
    fn = ops.gemv_gptq if kind == "gptq" else ops.gemv_awq
    y = fn(dev(torch, a), dev(torch, qw), dev(torch, scales16), dev(torch, qz), K, N,
           G).cpu().numpy()
    ofn = oracle.gptq if kind == "gptq" else oracle.awq
    W = gq_dense(q, zeros, scales16, G, kind)
    for b in range(B):
        ref = ofn(a[b].astype(np.float32), qw, scales16.astype(np.float32), qz, K, N, G)
        close(y[b], ref, a[b].astype(np.float32), W)
    # batch rows are independent: the last rows of the batched call equal a call on those
    # rows alone (batch 4 and up runs on MFMA, whose rows do not mix; batch 1 on the dot)
    t = 4 if B >= 4 else 1
    yt = fn(dev(torch, a[-t:]), dev(torch, qw), dev(torch, scales16), dev(torch, qz), K, N,
            G).cpu().numpy()
    np.testing.assert_array_equal(yt, y[-t:])


@pytest.mark.parametrize("kind", ["gptq", "awq"])
@pytest.mark.parametrize("B,K,N,G,f32s", [(4, 1024, 1000, 32, False), (5, 2048, 264, 64, True),
                                          (16, 4096, 96, 256, False), (9, 1536, 40, 512, False),
                                          (12, 2048, 520, 128, True), (6, 512, 72, 64, False)])
def test_gptq_awq_mfma_shapes(torch_dev, kind, B, K, N, G, f32s):
    """Batch 4-16 with fp16 activations runs on fp16 MFMA: ragged N (a partly used 32-column
    tile), batches that fill 4..16 of the 16 MFMA rows, every group size from 32 to 512
    (2..32 MFMA steps per group), fp16 and fp32 scales, K in 4, 2 and 1 parts per workgroup
    with one to three 512-k chunks per part."""
    from tenzo_amd import ops
    torch = torch_dev
    print(f"{kind} mfma B={B} K={K} N={N} G={G} f32s={f32s}", flush=True)
    rng = np.random.default_rng(B * 7 + K + N + G)
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    zeros = rng.integers(0, 16, size=(K // G, N), dtype=np.uint8)
    scales = synth.f16_round(np.abs(rng.normal(0, 0.01, size=(K // G, N))))
    scales = scales.astype(np.float32 if f32s else np.float16)
    pack = formats.gptq_pack if kind == "gptq" else formats.awq_pack
    qw, qz = pack(q, zeros)
    a = rng.standard_normal((B, K)).astype(np.float16)
    fn = ops.gemv_gptq if kind == "gptq" else ops.gemv_awq
    y = fn(dev(torch, a), dev(torch, qw), dev(torch, scales), dev(torch, qz), K, N,
           G).cpu().numpy()
    assert y.shape == (B, N)
    ofn = oracle.gptq if kind == "gptq" else oracle.awq
    W = gq_dense(q, zeros, scales, G, kind)
    for b in range(B):
        ref = ofn(a[b].astype(np.float32), qw, scales.astype(np.float32), qz, K, N, G)
        close(y[b], ref, a[b].astype(np.float32), W)


@pytest.mark.parametrize("kind", ["gptq", "awq"])
@pytest.mark.parametrize("B,K,N,G,f16a,f32s", [(1, 2048, 40, 32, True, False),
                                               (2, 6144, 1000, 64, False, True),
                                               (3, 4096, 520, 256, True, True),
                                               (4, 2048, 264, 128, False, False),
                                               (1, 4096, 8, 512, False, False),
                                               (2, 8192, 96, 1024, True, False),
                                               (4, 4096, 72, 1024, True, False),
                                               (1, 10240, 64, 128, True, False),
                                               (3, 3072, 128, 32, False, True)])
def test_gptq_awq_wide_load_shapes(torch_dev, kind, B, K, N, G, f16a, f32s):
    """Batch 1-4 on 128-bit weight loads (4 columns per lane): fp16 and fp32 activations and
    scales, groups of 32 (two per 64-k segment) up to 1024 (spanning several k-groups), one to
    three segments per k-group (K = 6144, 8192: two; 10240: three, the last k-group one),
    k-groups left without a segment (K = 2048, 3072), N not a multiple of the workgroup's 32
    columns, and batch 4 with fp16 activations where the MFMA path does not apply (group
    1024)."""
    from tenzo_amd import ops
    torch = torch_dev
    print(f"{kind} wide B={B} K={K} N={N} G={G} f16a={f16a} f32s={f32s}", flush=True)
    rng = np.random.default_rng(B * 13 + K + N + G)
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    zeros = rng.integers(0, 16, size=(K // G, N), dtype=np.uint8)
    scales = synth.f16_round(np.abs(rng.normal(0, 0.01, size=(K // G, N))))
    scales = scales.astype(np.float32 if f32s else np.float16)
    pack = formats.gptq_pack if kind == "gptq" else formats.awq_pack
    qw, qz = pack(q, zeros)
    a = rng.standard_normal((B, K)).astype(np.float16 if f16a else np.float32)
    fn = ops.gemv_gptq if kind == "gptq" else ops.gemv_awq
    y = fn(dev(torch, a), dev(torch, qw), dev(torch, scales), dev(torch, qz), K, N,
           G).cpu().numpy()
    assert y.shape == (B, N)
    ofn = oracle.gptq if kind == "gptq" else oracle.awq
    W = gq_dense(q, zeros, scales, G, kind)
    for b in range(B):
        a32 = a[b].astype(np.float32)
        close(y[b], ofn(a32, qw, scales.astype(np.float32), qz, K, N, G), a32, W)


def gq_dense(q, zeros, scales, G, kind):
    """[N][K] weights of GPTQ (zero = nibble + 1, :1117-1143) or AWQ (zero =
    nibble, :1146-1175) from the unpacked q [K][N], zeros and scales [K/G][N]."""
    z = zeros.astype(np.float64) + (1 if kind == "gptq" else 0)
    s = scales.astype(np.float64)
    return ((q.astype(np.float64) - np.repeat(z, G, axis=0)[:q.shape[0]]) *
            np.repeat(s, G, axis=0)[:q.shape[0]]).T


def test_gptq_fp32_scales_and_ragged_groups(torch_dev):
    from tenzo_amd import ops
    torch = torch_dev
    rng = np.random.default_rng(5)
    K, N, G = 640, 72, 128  # 5 groups: qzeros has a partly used second word row
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    zeros = rng.integers(0, 16, size=(K // G, N), dtype=np.uint8)
    scales = synth.f16_round(np.abs(rng.normal(0, 0.01, size=(K // G, N))))
    a = rng.standard_normal(K).astype(np.float32)
    qw, qz = formats.gptq_pack(q, zeros)
    y = ops.gemv_gptq(dev(torch, a), dev(torch, qw), dev(torch, scales), dev(torch, qz), K, N,
                      G).cpu().numpy()[0]
    close(y, oracle.gptq(a, qw, scales, qz, K, N, G), a, gq_dense(q, zeros, scales, G, "gptq"))
    qw, qz = formats.awq_pack(q, zeros)
    y = ops.gemv_awq(dev(torch, a), dev(torch, qw), dev(torch, scales), dev(torch, qz), K, N,
                     G).cpu().numpy()[0]
    close(y, oracle.awq(a, qw, scales, qz, K, N, G), a, gq_dense(q, zeros, scales, G, "awq"))
