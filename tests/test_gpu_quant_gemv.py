"""GGUF Q4_0 (fp16 / fp32 / Q8_0 activations), GPTQ and AWQ GEMVs on the GPU
against the CPU oracle and the compiled-reference goldens, at the benchmark
shapes (Q4_0 11008x4096; GPTQ/AWQ K=4096 N=14336 group 128, batch 1 and 8).
These are fp32 reductions in a different order from the reference, so the
bar is 1e-3 relative to the largest |y| of the call (outputs near zero are
sums of cancelling terms)."""
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


def close(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(y - ref).max() / np.abs(ref).max()
    print(f"  max err / max|y| = {err:.2e}", flush=True)
    assert err < RTOL


def make_q4(rng, N, K):
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    d = np.abs(rng.normal(0, 0.01, size=(N, K // 32))).astype(np.float16)
    return formats.q4_0_pack(q, d)


@pytest.mark.parametrize("N,K", [(64, 32), (100, 256), (11008, 4096), (257, 4128)])
def test_q4_0_fp16_and_fp32_activations(torch_dev, N, K):
    from tenzo_amd import ops
    torch = torch_dev
    print(f"q4_0 N={N} K={K}", flush=True)
    rng = np.random.default_rng(N + K)
    w = make_q4(rng, N, K)
    a16 = rng.standard_normal(K).astype(np.float16)
    ref = oracle.q4_0(a16.astype(np.float32), w, K, N)
    y = ops.gemv_q4_0(dev(torch, a16), dev(torch, w), K, N).cpu().numpy()[0]
    close(y, ref)
    y32 = ops.gemv_q4_0(dev(torch, a16.astype(np.float32)), dev(torch, w), K, N).cpu().numpy()[0]
    close(y32, ref)


@pytest.mark.parametrize("N,K", [(64, 32), (11008, 4096)])
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
    for b in range(B):
        ref = ofn(a[b].astype(np.float32), qw, scales16.astype(np.float32), qz, K, N, G)
        close(y[b], ref)
    # batch rows are independent: row b of the batched call equals a batch-1 call
    y1 = fn(dev(torch, a[-1:]), dev(torch, qw), dev(torch, scales16), dev(torch, qz), K, N,
            G).cpu().numpy()
    np.testing.assert_array_equal(y1[0], y[-1])


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
    close(y, oracle.gptq(a, qw, scales, qz, K, N, G))
    qw, qz = formats.awq_pack(q, zeros)
    y = ops.gemv_awq(dev(torch, a), dev(torch, qw), dev(torch, scales), dev(torch, qz), K, N,
                     G).cpu().numpy()[0]
    close(y, oracle.awq(a, qw, scales, qz, K, N, G))
