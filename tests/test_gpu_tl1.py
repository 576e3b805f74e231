"""TL1 GEMV and activation quantization on the GPU against the CPU oracle and
the compiled-reference golden vectors (bit-exact: int32 accumulators, int8
codes and the fp32 outputs, which are one multiply of them)."""
import ctypes
import os

import numpy as np
import pytest

import oracle
from tenzo_amd import formats

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU test needs a visible GPU"
    from tenzo_amd import _lib
    _lib.load()
    return torch


def to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def gpu_gemv(torch, w_tl1, x, N, K, w_scale, want_y=False):
    from tenzo_amd import ops
    wp = ops.tl1_repack(to_dev(torch, w_tl1), N, K)
    codes, q, _ = ops.rmsnorm_quant31(to_dev(torch, x), None)
    y, acc = ops.bitlinear_tl1(codes, q, wp, w_scale, N, K, want_acc=True)
    torch.cuda.synchronize()
    return (y.cpu().numpy()[0], acc.cpu().numpy()[0], codes.cpu().numpy()[0, :K],
            ops.actq_inv_scale(q).cpu().numpy()[0], q[:, 1].cpu().numpy()[0])


def test_tl1_gemv_matches_reference_goldens(torch_dev):
    z = np.load(os.path.join(GOLD, "tl1_gemv.npz"))
    for tag in "abc":
        w, x = z[f"{tag}_w"], z[f"{tag}_x"]
        N, K = z[f"{tag}_tern"].shape
        print(f"golden {tag}: N={N} K={K}", flush=True)
        y, acc, codes, inv, csum = gpu_gemv(torch_dev, w, x, N, K, float(z[f"{tag}_w_scale"]))
        np.testing.assert_array_equal(acc, z[f"{tag}_acc"])
        assert inv.view(np.uint32) == z[f"{tag}_inv"].view(np.uint32)
        np.testing.assert_array_equal(y.view(np.uint32), z[f"{tag}_y"].view(np.uint32))
        np.testing.assert_array_equal(oracle.build_lut(codes), z[f"{tag}_lut"])
        assert csum == int(codes.astype(np.int64).sum())


@pytest.mark.parametrize("N,K", [(64, 2), (64, 64), (128, 130), (192, 1000), (6912, 2560),
                                 (2560, 6912), (3840, 2560)])
def test_tl1_gemv_matches_oracle(torch_dev, N, K):
    print(f"tl1 N={N} K={K}", flush=True)
    rng = np.random.default_rng(N * 7 + K)
    w = formats.tl1_random(N, K, rng)
    x = rng.standard_normal(K).astype(np.float32)
    y, acc, codes, inv, _ = gpu_gemv(torch_dev, w, x, N, K, 0.0159)
    yo, acco, invo = oracle.tl1_gemv(x, w, N, 0.0159)
    np.testing.assert_array_equal(acc, acco)
    np.testing.assert_array_equal(y, yo)
    assert inv == invo


def test_tl1_gemv_batched_rows(torch_dev):
    from tenzo_amd import ops
    torch = torch_dev
    rng = np.random.default_rng(3)
    N, K, M = 256, 640, 3
    w = formats.tl1_random(N, K, rng)
    x = rng.standard_normal((M, K)).astype(np.float32)
    wp = ops.tl1_repack(to_dev(torch, w), N, K)
    y = ops.bitlinear_tl1_f32(to_dev(torch, x), wp, 0.02, N, K).cpu().numpy()
    for m in range(M):
        yo, _, _ = oracle.tl1_gemv(x[m], w, N, 0.02)
        np.testing.assert_array_equal(y[m], yo)


@pytest.mark.parametrize("N,K,M", [(6912, 2560, 1), (192, 2500, 2), (64, 1000, 1),
                                   (2560, 6912, 1), (128, 102, 1)])
def test_tl1_gemv_f32_entry_bit_exact(torch_dev, N, K, M):
    """tenzo_hip_bitlinear_tl1_f32 (fp32 activations in: build_lut's
    quantization, then the GEMV) against the oracle, bit for bit: the fused
    one-launch kernel (6912 x 2560 = BASELINE config 1; K not a multiple of
    64; two rows) and the two-launch path (K split by the GEMV, K % 4 != 0).
    Row 0 of the two-row case is all zeros (the 1e-6 absmax floor, codes 0)."""
    from tenzo_amd import ops
    torch = torch_dev
    rng = np.random.default_rng(N + K)
    w = formats.tl1_random(N, K, rng)
    x = rng.standard_normal((M, K)).astype(np.float32)
    if M > 1:
        x[0] = 0.0
    wp = ops.tl1_repack(to_dev(torch, w), N, K)
    print(f"tl1_f32 N={N} K={K} M={M}", flush=True)
    y = ops.bitlinear_tl1_f32(to_dev(torch, x), wp, 0.0159, N, K).cpu().numpy()
    for m in range(M):
        yo, _, _ = oracle.tl1_gemv(x[m], w, N, 0.0159)
        np.testing.assert_array_equal(y[m], yo)


def test_rmsnorm_quant31_bit_exact(torch_dev):
    from tenzo_amd import ops
    torch = torch_dev
    rng = np.random.default_rng(4)
    # 16384: the longest row the register path holds; 16390, 20001: rows past
    # the LDS chain layout (chains read from memory); 101: K % 4 != 0
    for K in (2560, 6912, 100, 101, 16384, 16390, 20001):
        print(f"rmsnorm_quant31 K={K}", flush=True)
        x = (rng.standard_normal(K) * 3).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
        codes, q, y = ops.rmsnorm_quant31(to_dev(torch, x), to_dev(torch, w), want_y=True)
        y = y.cpu().numpy()[0]
        yo = oracle.rms_norm(x, w)
        np.testing.assert_array_equal(y, yo)  # the reference build's arithmetic, as the oracle
        co, invo = oracle.quant31(yo)
        np.testing.assert_array_equal(codes.cpu().numpy()[0, :K], co)
        assert not codes.cpu().numpy()[0, K:].any()
        assert ops.actq_inv_scale(q).cpu().numpy()[0] == invo
        yn = ops.rmsnorm(to_dev(torch, x), None).cpu().numpy()
        np.testing.assert_array_equal(yn, oracle.rms_norm(x, None))


def test_rmsnorm_against_reference_goldens(torch_dev):
    from tenzo_amd import ops
    torch = torch_dev
    from tests.golden.make_golden import RMS_DIMS
    z = np.load(os.path.join(GOLD, "rmsnorm.npz"))
    for dim in RMS_DIMS:
        print(f"rmsnorm golden dim={dim}", flush=True)
        y = ops.rmsnorm(to_dev(torch, z[f"x{dim}"]), to_dev(torch, z[f"w{dim}"])).cpu().numpy()
        np.testing.assert_array_equal(y, z[f"y{dim}"])
        y0 = ops.rmsnorm(to_dev(torch, z[f"x{dim}"]), None).cpu().numpy()
        np.testing.assert_array_equal(y0, z[f"ynow{dim}"])


def test_host_pointer_shims(torch_dev):
    from tenzo_amd import _lib
    L = _lib.load()
    rng = np.random.default_rng(5)
    N, K = 128, 256
    w = formats.tl1_random(N, K, rng)
    x = rng.standard_normal((2, K)).astype(np.float32)
    y = np.empty((2, N), np.float32)
    P = lambda a: ctypes.c_void_p(a.ctypes.data)  # noqa: E731
    assert L.tenzo_hip_execute_bitlinear_tl1(P(x), P(w), P(y), 2, K, N, 0.5) == 1
    for m in range(2):
        np.testing.assert_array_equal(y[m], oracle.tl1_gemv(x[m], w, N, 0.5)[0])
    xn = rng.standard_normal(K).astype(np.float32)
    wn = rng.standard_normal(K).astype(np.float32)
    yn = np.empty(K, np.float32)
    assert L.tenzo_hip_execute_rmsnorm(P(xn), P(wn), P(yn), K, 1e-5) == 1
    np.testing.assert_array_equal(yn, oracle.rms_norm(xn, wn))
    # bad arguments are rejected, not run
    assert L.tenzo_hip_execute_bitlinear_tl1(P(x), P(w), P(y), 2, K, 100, 0.5) == 0


@pytest.mark.parametrize("N,K,M", [(64, 2, 1), (128, 130, 1), (6912, 2560, 1), (2560, 6912, 1),
                                   (256, 640, 3)])
def test_tl1_lut_gemv_equals_dot4_gemv(torch_dev, N, K, M):
    """The table-method kernel (the reference's build_lut / pshufb lookup on
    the GPU) gives the masked-v_dot4 kernel's int32 sums and outputs bit for
    bit, and the oracle's."""
    from tenzo_amd import ops
    torch = torch_dev
    print(f"tl1 lut N={N} K={K} M={M}", flush=True)
    rng = np.random.default_rng(N + 3 * K + M)
    w = formats.tl1_random(N, K, rng)
    x = rng.standard_normal((M, K)).astype(np.float32)
    wp = ops.tl1_repack(to_dev(torch, w), N, K)
    codes, q, _ = ops.rmsnorm_quant31(to_dev(torch, x), None)
    y, acc = ops.bitlinear_tl1(codes, q, wp, 0.0159, N, K, want_acc=True)
    yl, accl = ops.bitlinear_tl1_lut(codes, q, wp, 0.0159, N, K, want_acc=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(accl.cpu().numpy(), acc.cpu().numpy())
    np.testing.assert_array_equal(yl.cpu().numpy().view(np.uint32), y.cpu().numpy().view(np.uint32))
    yo, acco, _ = oracle.tl1_gemv(x[0], w, N, 0.0159)
    np.testing.assert_array_equal(accl.cpu().numpy()[0], acco)
