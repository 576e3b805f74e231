"""int8 LM head, greedy argmax, repetition penalty and embedding lookup on the
GPU against the CPU oracle: logits are one fp32 multiply of an exact int32
dot, so they are compared bit for bit."""
import numpy as np
import pytest

import oracle
from tenzo_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU test needs a visible GPU"
    from tenzo_amd import _lib
    _lib.load()
    return torch


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("V,H", [(64, 16), (65, 32), (1000, 512), (4096, 2560), (128256, 2560)])
def test_lm_head_i8_matches_oracle(torch_dev, V, H):
    from tenzo_amd import ops
    torch = torch_dev
    print(f"lm_head V={V} H={H}", flush=True)
    rng = np.random.default_rng(V + H)
    if V * H > 50_000_000:  # large table: random codes / scales of the same ranges
        W = rng.integers(-127, 128, size=(V, H), dtype=np.int8)
        s = rng.uniform(2e-4, 8e-4, size=V).astype(np.float32)
    else:
        W, s = synth.head_quantize(rng.normal(0, 0.02, size=(V, H)).astype(np.float32))
    x = (rng.standard_normal(H) * 2).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    wp = ops.i8_rows_repack(dev(torch, W), V, H)
    logits = ops.lm_head_i8(dev(torch, x), dev(torch, nw), wp, dev(torch, s), V, H).cpu().numpy()
    xn = oracle.rms_norm(x, nw)
    ref, _, _ = oracle.lm_head(xn, W, s)
    np.testing.assert_array_equal(logits.view(np.uint32), ref.view(np.uint32))
    idx = ops.argmax(dev(torch, logits)).cpu().numpy()[0]
    assert idx == oracle.argmax(ref)


def test_argmax_first_maximum_and_ties(torch_dev):
    from tenzo_amd import ops
    torch = torch_dev
    rng = np.random.default_rng(1)
    for V in (1, 7, 4096, 4097, 128256, 300000):
        print(f"argmax V={V}", flush=True)
        lg = rng.standard_normal(V).astype(np.float32)
        assert ops.argmax(dev(torch, lg)).cpu().numpy()[0] == oracle.argmax(lg)
        if V > 10:
            lg[V // 3] = lg[V - 2] = lg[5] = 100.0  # three equal maxima: the first wins
            assert ops.argmax(dev(torch, lg)).cpu().numpy()[0] == 5
    lg = np.full(5000, -np.inf, np.float32)
    assert ops.argmax(dev(torch, lg)).cpu().numpy()[0] == 0


def test_embed_i8_bit_exact(torch_dev):
    from tenzo_amd import ops
    torch = torch_dev
    rng = np.random.default_rng(2)
    V, H = 300, 256
    W, s = synth.head_quantize(rng.normal(0, 0.02, size=(V, H)).astype(np.float32))
    wp = ops.i8_rows_repack(dev(torch, W), V, H)
    ts = dev(torch, s)
    for tok in (0, 63, 64, 299):
        x = ops.embed_i8(wp, ts, dev(torch, np.array([tok], np.int32)), V, H).cpu().numpy()
        ref = np.empty(H, np.float32)
        oracle.lib().orc_embed_i8(oracle._ptr(W), oracle._ptr(s), H, tok, oracle._ptr(ref))
        np.testing.assert_array_equal(x, ref)
    # an out-of-range token reads nothing and gives zeros
    x = ops.embed_i8(wp, ts, dev(torch, np.array([V], np.int32)), V, H).cpu().numpy()
    assert not x.any()


def test_packed_layout_roundtrip(torch_dev):
    """The packed table holds row r's 16-column chunk c at ((r/64)*(H/16)+c)*64+r%64."""
    from tenzo_amd import ops
    torch = torch_dev
    rng = np.random.default_rng(3)
    V, H = 130, 48
    W = rng.integers(-128, 128, size=(V, H), dtype=np.int8)
    p = ops.i8_rows_repack(dev(torch, W), V, H).cpu().numpy().view(np.int8)
    nb = (V + 63) // 64
    blocks = p.reshape(nb, H // 16, 64, 16)
    full = np.zeros((nb * 64, H), np.int8)
    full[:V] = W
    np.testing.assert_array_equal(blocks.transpose(0, 2, 1, 3).reshape(nb * 64, H), full)
