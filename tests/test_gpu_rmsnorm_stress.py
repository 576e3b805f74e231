"""RMSNorm on the GPU against the oracle's restatement of the reference build
(eight sequential FMA chains, RSQRTSS estimate + Newton step, (x*w)*inv) on
rows built to stress the kernels' parallel evaluation of the chains: values
with few mantissa bits (rounding ties are possible at every step), magnitudes
spread over many binades, sparse rows, a single spike, near-constant rows and
tiny values (grids below the normal range), at the model's dims and ragged
ones. Every output must be bit-exact."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def rows(kind, M, K, rng):
    v = rng.standard_normal((M, K)).astype(np.float32)
    if kind == 1:  # 11-bit mantissas
        u = v.view(np.uint32)
        v = ((u + np.uint32(0x1000)) & np.uint32(0xFFFFE000)).view(np.float32)
    elif kind == 2:
        v = (v * np.exp(6.0 * rng.standard_normal((M, K)))).astype(np.float32)
    elif kind == 3:
        v = (np.round(v * 4) / 4).astype(np.float32)
    elif kind == 4:
        v[rng.random((M, K)) < 0.9] = 0
    elif kind == 5:
        v *= np.float32(1e-3)
        v[:, K // 3] = 1000
    elif kind == 6:
        v = (1 + 0.01 * v).astype(np.float32)
    elif kind == 7:
        v = (v * np.float32(1e-20)).astype(np.float32)
    return np.ascontiguousarray(v, np.float32)


@pytest.mark.parametrize("K", [2560, 6912, 8192, 64, 100, 16384, 7, 20001])
def test_rmsnorm_stress_bit_exact(K):
    import torch
    assert torch.cuda.is_available(), "GPU test needs a visible GPU"
    from tenzo_amd import ops
    rng = np.random.default_rng(K)
    M = 24 if K > 8192 else 48
    w = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    tw = torch.from_numpy(w).cuda()
    for kind in range(8):
        print(f"rmsnorm stress K={K} kind={kind}", flush=True)
        x = rows(kind, M, K, rng)
        tx = torch.from_numpy(x).cuda()
        # rows held in registers (K % 4 == 0, K <= 16384) or streamed
        _, _, y = ops.rmsnorm_quant31(tx, tw, want_y=True)
        y = y.cpu().numpy()
        for m in range(M):
            np.testing.assert_array_equal(y[m], oracle.rms_norm(x[m], w),
                                          err_msg=f"K {K} kind {kind} row {m}")
        # the single-row operator (executeRMSNorm), without weights
        for m in range(0, M, 8):
            yn = ops.rmsnorm(tx[m].contiguous(), None).cpu().numpy()
            np.testing.assert_array_equal(yn, oracle.rms_norm(x[m], None),
                                          err_msg=f"K {K} kind {kind} row {m} (no weight)")
