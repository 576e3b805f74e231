"""Multi-token TL1 contraction on int8 MFMA (prefill) against the per-token
GEMV and the CPU oracle: the int32 accumulators are exact, so the batched
results equal the sequential per-token ones bit for bit (fp32 outputs are one
multiply of them)."""
import numpy as np
import pytest

import oracle
from tenzo_amd import formats

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU test needs a visible GPU"
    from tenzo_amd import _lib
    _lib.load()
    return torch


def to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _setup(torch, N, K, M, seed):
    from tenzo_amd import ops
    rng = np.random.default_rng(seed)
    w = formats.tl1_random(N, K, rng)
    x = (rng.standard_normal((M, K)) * rng.uniform(0.1, 10, (M, 1))).astype(np.float32)
    wp = ops.tl1_repack(to_dev(torch, w), N, K)
    codes, q, _ = ops.rmsnorm_quant31(to_dev(torch, x), None)
    return w, x, wp, codes, q


@pytest.mark.parametrize("N,K", [(64, 64), (128, 130), (192, 1000), (3840, 2560),
                                 (2560, 6912), (13824, 2560)])
@pytest.mark.parametrize("M", [1, 7, 16, 33, 64, 100])
def test_batch_equals_per_token_gemv(torch_dev, N, K, M):
    from tenzo_amd import ops
    torch = torch_dev
    print(f"tl1_batch N={N} K={K} M={M}", flush=True)
    w, x, wp, codes, q = _setup(torch, N, K, M, N + 3 * K + 7 * M)
    yb, ab = ops.bitlinear_tl1_batch(codes, q, wp, 0.0173, N, K, want_acc=True)
    yg, ag = ops.bitlinear_tl1(codes, q, wp, 0.0173, N, K, want_acc=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ab.cpu().numpy(), ag.cpu().numpy())
    np.testing.assert_array_equal(yb.cpu().numpy().view(np.uint32),
                                  yg.cpu().numpy().view(np.uint32))
    # the first and last token against the oracle, from the CPU quantization
    for m in sorted({0, M - 1}):
        yo, acco, _ = oracle.tl1_gemv(x[m], w, N, 0.0173)
        np.testing.assert_array_equal(ab[m].cpu().numpy(), acco)
        np.testing.assert_array_equal(yb[m].cpu().numpy(), yo)


@pytest.mark.parametrize("tile", [142, 242, 442, 222, 422, 221, 421, 412, 411, 811])
def test_batch_every_tile_shape(torch_dev, tile):
    """Every workgroup tile shape gives the same exact sums, with a ragged
    token count and a K that is not a multiple of the chunk (64) or of the
    K groups' runs."""
    from tenzo_amd import ops
    torch = torch_dev
    N, K, M = 1280, 2600, 70
    print(f"tl1_batch tile={tile}", flush=True)
    w, x, wp, codes, q = _setup(torch, N, K, M, 11)
    ref, _ = ops.bitlinear_tl1(codes, q, wp, 0.5, N, K)
    for _ in range(2):
        yb, _ = ops.bitlinear_tl1_batch(codes, q, wp, 0.5, N, K, tile=tile)
        np.testing.assert_array_equal(yb.cpu().numpy(), ref.cpu().numpy())


def test_batch_prompt_sized(torch_dev):
    """A 512-token prompt at the largest projection: every row against the
    per-token GEMV, a sample against the oracle's integer contraction."""
    from tenzo_amd import ops
    torch = torch_dev
    N, K, M = 13824, 2560, 512
    w, x, wp, codes, q = _setup(torch, N, K, M, 5)
    yb, ab = ops.bitlinear_tl1_batch(codes, q, wp, 1.0, N, K, want_acc=True)
    _, ag = ops.bitlinear_tl1(codes, q, wp, 1.0, N, K, want_acc=True)
    assert torch.equal(ab, ag)
    c = codes.cpu().numpy()
    for m in (0, 255, 511):
        acc = oracle.tl1_gemv_i32(w, c[m, :K], N, K)
        np.testing.assert_array_equal(ab[m].cpu().numpy(), acc)


def test_batch_zero_and_extreme_codes(torch_dev):
    """All-zero rows (absmax floor) and rows at the code range limits."""
    from tenzo_amd import ops
    torch = torch_dev
    N, K, M = 256, 640, 20
    rng = np.random.default_rng(2)
    w = formats.tl1_random(N, K, rng)
    x = np.zeros((M, K), np.float32)
    x[1] = 1e30
    x[2] = -3.0
    x[3, ::2] = 7.0
    x[3, 1::2] = -7.0
    x[4:] = rng.standard_normal((M - 4, K))
    wp = ops.tl1_repack(to_dev(torch, w), N, K)
    codes, q, _ = ops.rmsnorm_quant31(to_dev(torch, x), None)
    yb, ab = ops.bitlinear_tl1_batch(codes, q, wp, 0.25, N, K, want_acc=True)
    for m in range(M):
        yo, acco, _ = oracle.tl1_gemv(x[m], w, N, 0.25)
        np.testing.assert_array_equal(ab[m].cpu().numpy(), acco)
        np.testing.assert_array_equal(yb[m].cpu().numpy(), yo)
