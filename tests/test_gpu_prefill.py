"""Multi-token prefill: the TL1 contraction on int8 MFMA against the
per-token GEMV and the CPU oracle (the int32 accumulators are exact, so the
batched results equal the sequential per-token ones bit for bit: fp32 outputs
are one multiply of them), and the engine's batched prefill against one
prefill_token call per token (KV cache, hidden state and the following
decode steps bit for bit: every stage runs the same arithmetic)."""
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


def _engine_pair(eng_mod, cfg, sm):
    a, b = eng_mod.Engine(cfg), eng_mod.Engine(cfg)
    for e in (a, b):
        e.set_model(sm)
        e.set_mode("eager")
    return a, b


@pytest.mark.parametrize("ctx,n", [(0, 1), (0, 5), (0, 40), (5, 23), (17, 30)])
def test_engine_prefill_equals_token_by_token(torch_dev, ctx, n):
    """exact=True: one pass of the batched pipeline equals n prefill_token
    calls of the per-stage (eager) path bit for bit."""
    from tenzo_amd import engine as eng_mod, synth
    cfg = synth.DecodeConfig(hidden=512, n_q_heads=4, n_kv_heads=1, n_layers=3, ffn=1024,
                             vocab=2048, max_seq=64, theta=10000.0)
    sm = synth.make_model(cfg, seed=61 + n, ctx=ctx)
    rng = np.random.default_rng(n)
    toks = rng.integers(0, cfg.vocab, n).astype(np.int32)
    print(f"engine prefill ctx={ctx} n={n}", flush=True)
    a, b = _engine_pair(eng_mod, cfg, sm)
    with a, b:
        for t in toks:
            a.prefill(int(t))
        b.prefill_batch(toks, exact=True)
        assert a.seq_len == b.seq_len == ctx + n
        for x, y in zip(a.get_kv(ctx + n), b.get_kv(ctx + n)):
            np.testing.assert_array_equal(x, y)
        np.testing.assert_array_equal(a.buffer("x"), b.buffer("x"))
        for t in (7, 11, 13):
            assert a.step(t) == b.step(t)
            np.testing.assert_array_equal(a.logits(), b.logits())


def test_engine_prefill_longer_than_one_pass(torch_dev):
    """600 tokens: two passes of the 512-row buffers, attention over up to 19
    chunks per query, G = 4 query heads per kv head."""
    from tenzo_amd import engine as eng_mod, synth
    cfg = synth.DecodeConfig(hidden=512, n_q_heads=4, n_kv_heads=1, n_layers=2, ffn=512,
                             vocab=1024, max_seq=640, theta=10000.0)
    sm = synth.make_model(cfg, seed=71, ctx=0)
    toks = np.random.default_rng(3).integers(0, cfg.vocab, 600).astype(np.int32)
    a, b = _engine_pair(eng_mod, cfg, sm)
    with a, b:
        for t in toks:
            a.prefill(int(t))
        b.prefill_batch(toks, exact=True)
        for x, y in zip(a.get_kv(600), b.get_kv(600)):
            np.testing.assert_array_equal(x, y)
        np.testing.assert_array_equal(a.buffer("x"), b.buffer("x"))
        assert a.step(5) == b.step(5)
        np.testing.assert_array_equal(a.logits(), b.logits())


def test_engine_prefill_chunk_size_changes(torch_dev):
    """16 kv heads: decode aims at 512 / 16 = 32 chunks per head, so its chunk
    size is 32 tokens up to a context of 1024 and 64 past it (ceil(ctx / 32)
    rounded up to a multiple of 32); a prompt from position 1000 mixes both
    in one launch (rows with 32-token chunks run in the kernel built for 64),
    G = 1."""
    from tenzo_amd import engine as eng_mod, synth
    cfg = synth.DecodeConfig(hidden=2048, n_q_heads=16, n_kv_heads=16, n_layers=1, ffn=512,
                             vocab=512, max_seq=1100, theta=10000.0)
    sm = synth.make_model(cfg, seed=29, ctx=1000)
    toks = np.random.default_rng(4).integers(0, cfg.vocab, 60).astype(np.int32)
    print("engine prefill ctx=1000 n=60 Hkv=16", flush=True)
    a, b = _engine_pair(eng_mod, cfg, sm)
    with a, b:
        for t in toks:
            a.prefill(int(t))
        b.prefill_batch(toks, exact=True)
        for x, y in zip(a.get_kv(1060), b.get_kv(1060)):
            np.testing.assert_array_equal(x, y)
        np.testing.assert_array_equal(a.buffer("x"), b.buffer("x"))
        assert a.step(9) == b.step(9)
        np.testing.assert_array_equal(a.logits(), b.logits())


@pytest.mark.parametrize("ctx", [2020, 3180])
def test_engine_prefill_wide_merge(torch_dev, ctx):
    """One kv head: decode aims at 512 chunks per head, so its chunks stay 32
    tokens long; past a chunk count the merge moves to the four-group kernel
    (attn_combine_wide_kernel). A prompt of 60 tokens from position 2020 (64 ->
    65 chunks) puts rows on both sides of that line in one launch, one from
    3180 (100 -> 102) only past it; the exact prefill must still equal
    token-by-token decode bit for bit."""
    from tenzo_amd import engine as eng_mod, synth
    cfg = synth.DecodeConfig(hidden=512, n_q_heads=4, n_kv_heads=1, n_layers=1, ffn=512,
                             vocab=512, max_seq=3300, theta=10000.0)
    sm = synth.make_model(cfg, seed=37, ctx=ctx)
    toks = np.random.default_rng(6).integers(0, cfg.vocab, 60).astype(np.int32)
    print(f"engine prefill ctx={ctx} n=60 Hkv=1", flush=True)
    a, b = _engine_pair(eng_mod, cfg, sm)
    with a, b:
        for t in toks:
            a.prefill(int(t))
        b.prefill_batch(toks, exact=True)
        for x, y in zip(a.get_kv(ctx + 60), b.get_kv(ctx + 60)):
            np.testing.assert_array_equal(x, y)
        np.testing.assert_array_equal(a.buffer("x"), b.buffer("x"))
        assert a.step(9) == b.step(9)
        np.testing.assert_array_equal(a.logits(), b.logits())


def test_engine_prefill_then_persistent_decode(torch_dev):
    """A batched prefill followed by persistent-kernel decode steps gives the
    tokens of token-by-token prefill + decode (fp32 logits to 1e-5: the
    persistent kernel sums attention in its own order)."""
    from tenzo_amd import engine as eng_mod, synth
    cfg = synth.DecodeConfig(hidden=512, n_q_heads=4, n_kv_heads=1, n_layers=3, ffn=1024,
                             vocab=2048, max_seq=64, theta=10000.0)
    sm = synth.make_model(cfg, seed=83, ctx=0)
    toks = np.arange(1, 20, dtype=np.int32) * 37 % cfg.vocab
    with eng_mod.Engine(cfg) as a, eng_mod.Engine(cfg) as b:
        a.set_model(sm)
        b.set_model(sm)
        for t in toks:
            a.prefill(int(t))
        b.prefill_batch(toks, exact=True)
        ta, tb = a.decode(3, 6)[0], b.decode(3, 6)[0]
        assert list(ta) == list(tb)
        la, lb = a.logits(), b.logits()
        assert np.abs(la - lb).max() <= 1e-5 * max(np.abs(la).max(), 1e-30)


def test_engine_prefill_errors(torch_dev):
    from tenzo_amd import engine as eng_mod, synth
    cfg = synth.DecodeConfig(hidden=512, n_q_heads=4, n_kv_heads=1, n_layers=1, ffn=512,
                             vocab=256, max_seq=16, theta=10000.0)
    sm = synth.make_model(cfg, seed=5, ctx=0)
    with eng_mod.Engine(cfg) as e:
        e.set_model(sm)
        with pytest.raises(RuntimeError, match="outside"):
            e.prefill_batch(np.array([1, 256], np.int32))
        with pytest.raises(RuntimeError, match="full"):
            e.prefill_batch(np.zeros(17, np.int32))
        assert e.seq_len == 0
        e.prefill_batch(np.zeros(16, np.int32))
        assert e.seq_len == 16


@pytest.mark.parametrize("ctx,n,G", [(0, 40, 4), (17, 47, 4), (0, 600, 4), (3, 130, 1),
                                     (0, 70, 2)])
def test_engine_prefill_streaming_attention(torch_dev, ctx, n, G):
    """The default (streaming attention) prefill against the exact one: the
    attention differs only in how the softmax sums are grouped, so the hidden
    state agrees to 1e-4 and almost every KV code is identical (a code can flip
    where a value sits on a rounding boundary). The next decode step (on the
    persistent kernel, whose per-layer int32 sums are read back) attends over
    those caches: when every layer's activation codes are the same in both
    engines (every TL1 sum equal) the new hidden states agree to 1e-4; a +-31
    code can flip at a rounding tie, which moves them by ~1e-3, and only then
    -- exactly one GEMV whose sums differ, each by at most one weight (a
    single code moved by one) -- are they held to 1e-2. Each engine's logits
    must equal, bit for bit, the oracle's LM head applied to its own hidden
    state (the head's +-127 codes may flip at ties between the two engines,
    but never between an engine and the oracle). The greedy token must agree."""
    from tenzo_amd import engine as eng_mod, synth
    cfg = synth.DecodeConfig(hidden=512, n_q_heads=4, n_kv_heads=4 // G, n_layers=2, ffn=512,
                             vocab=1024, max_seq=ctx + n + 8, theta=10000.0)
    sm = synth.make_model(cfg, seed=97 + n, ctx=ctx)
    toks = np.random.default_rng(n).integers(0, cfg.vocab, n).astype(np.int32)
    print(f"streaming prefill ctx={ctx} n={n} G={G}", flush=True)
    a, b = _engine_pair(eng_mod, cfg, sm)
    with a, b:
        a.prefill_batch(toks, exact=True)
        b.prefill_batch(toks)
        xa, xb = a.buffer("x"), b.buffer("x")
        assert rel(xb, xa) < 1e-4
        for u, v in zip(a.get_kv(ctx + n), b.get_kv(ctx + n)):
            u, v = np.asarray(u, np.float64), np.asarray(v, np.float64)
            assert (u != v).mean() < 0.01
        a.set_mode("persistent")
        b.set_mode("persistent")
        ta, tb = a.step(5), b.step(5)
        la, lb = a.logits(), b.logits()
        moved = []
        for l in range(cfg.n_layers):
            for name in ("acc_qkv", "acc_o", "acc_gu", "acc_down"):
                d = a.layer_state(l, name).astype(np.int64) - b.layer_state(l, name)
                if d.any():
                    moved.append((l, name, int(np.abs(d).max())))
        # the head is exact given its input: each engine's logits equal the
        # oracle's LM head (bit-exact rms_norm, +-127 codes, int8 rows) applied
        # to that engine's own final hidden state
        xa2, xb2 = a.buffer("x"), b.buffer("x")
        for x, lg in ((xa2, la), (xb2, lb)):
            ref_lg = oracle.lm_head(oracle.rms_norm(x, sm.final_norm), sm.embed,
                                    sm.embed_scales)[0]
            np.testing.assert_array_equal(lg, ref_lg)
        print(f"GEMVs whose sums differ: {moved}; hidden rel {rel(xb2, xa2):.2e}", flush=True)
        if not moved:
            assert rel(xb2, xa2) < 1e-4
        else:
            assert len(moved) == 1 and moved[0][2] == 1, moved
            assert rel(xb2, xa2) < 1e-2
        assert ta == tb


def rel(a, b):
    return np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30)
