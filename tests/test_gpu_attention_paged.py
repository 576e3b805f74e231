"""paged_int8 on the GPU: the decode attention op against the CPU oracle and
the compiled reference's fixture (permuted block tables, the 1e-7 cut-off), and
the engine with kv_mode paged_int8 against the oracle's decode step and the
reference engine's own greedy steps and block table.

Bars: pool rows and scales bit-exact, op outputs 1e-5 relative (fp32 sums in
another order); chained engine steps 1e-3 on the hidden state and logits with
the greedy tokens equal (as for int8_fused)."""
import os

import numpy as np
import pytest

import oracle
from tenzo_amd import synth
from tests.golden.make_golden import TINY, load_tiny_model

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU test needs a visible GPU"
    from tenzo_amd import _lib
    _lib.load()
    return torch


def rel(a, b):
    return np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30)


def run_gpu(torch, q, k, v, pools, bt, layer, pos):
    from tenzo_amd import ops
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    t = [dev(a) for a in pools]
    cs = ops.rope_table(10000.0, pos, 1)[0].cuda()
    out = ops.attn_paged_int8_decode(dev(q), dev(k), dev(v), *t, dev(np.asarray(bt, np.int32)),
                                     layer, cs, pos)
    torch.cuda.synchronize()
    return out.cpu().numpy()[0], [a.cpu().numpy() for a in t]


@pytest.mark.parametrize("Hq,Hkv,L,layer,S,pos,qs", [
    (4, 1, 1, 0, 64, 0, 1.0), (8, 2, 3, 1, 320, 37, 1.0), (20, 5, 2, 1, 640, 600, 1.0),
    (16, 2, 1, 0, 2048, 2000, 1.0), (8, 8, 1, 0, 256, 47, 1.0), (8, 2, 2, 1, 320, 64, 1.0),
    (4, 2, 1, 0, 4096, 4095, 1.0), (8, 2, 2, 0, 640, 500, 40.0)])
def test_attn_paged_matches_oracle(torch_dev, Hq, Hkv, L, layer, S, pos, qs):
    print(f"attn_paged Hq={Hq} Hkv={Hkv} L={L} layer={layer} S={S} pos={pos} qs={qs}", flush=True)
    cfg = synth.DecodeConfig(hidden=Hq * 128, n_q_heads=Hq, n_kv_heads=Hkv, n_layers=L, ffn=64,
                             vocab=64, max_seq=S, theta=10000.0)
    nb = (S + 15) // 16
    rng = np.random.default_rng(pos + 7)
    bt = rng.permutation(nb).astype(np.int32)
    pools = synth.paged_kv(cfg, pos, bt, seed=pos)
    q = (qs * rng.standard_normal(Hq * 128)).astype(np.float32)
    k = (2 * rng.standard_normal(Hkv * 128)).astype(np.float32)
    v = rng.standard_normal(Hkv * 128).astype(np.float32)
    out, got = run_gpu(torch_dev, q, k, v, pools, bt, layer, pos)
    ref = [a.copy() for a in pools]
    o_ref, _, _ = oracle.attention_step_paged(q, k, v, *ref, bt, L, layer, Hq, Hkv, pos,
                                              oracle.rope_table(10000.0, pos))
    for a, b in zip(got, ref):
        np.testing.assert_array_equal(a, b)
    assert rel(out, o_ref) < 1e-5


@pytest.mark.parametrize("case", ["", "peak_"])
def test_attn_paged_reference_fixture(torch_dev, case):
    z = np.load(os.path.join(GOLD, "attention_paged.npz"))
    pools = [z[n] for n in ("pk", "pv", "pks", "pvs")]
    out, got = run_gpu(torch_dev, z[case + "q"], z[case + "k"], z[case + "v"], pools,
                       z[case + "block_table"], 1, 96)
    for a, n in zip(got, ("pk", "pv", "pks", "pvs")):
        np.testing.assert_array_equal(a, z[case + n + "_out"])
    assert rel(out, z[case + "out"]) < 1e-5


CFG = synth.DecodeConfig(hidden=512, n_q_heads=4, n_kv_heads=2, n_layers=3, ffn=1024,
                         vocab=2048, max_seq=640, theta=10000.0)


def to_pools(sm, cfg):
    """The model's logical cache placed in blocks 0, 1, ... (the engine's block
    manager allocates them in that order from a reset)."""
    nb = (cfg.max_seq + 15) // 16
    ident = np.arange(nb, dtype=np.int32)
    pk = np.zeros((nb, cfg.n_layers, cfg.n_kv_heads, 16, 128), np.int8)
    pv = np.zeros_like(pk)
    pks = np.ones((nb, cfg.n_layers, cfg.n_kv_heads, 16), np.float32)
    pvs = np.ones_like(pks)
    for t in range(sm.ctx):
        pk[t // 16, :, :, t % 16] = sm.kc[:, :, t]
        pv[t // 16, :, :, t % 16] = sm.vc[:, :, t]
        pks[t // 16, :, :, t % 16] = sm.ks[:, :, t]
        pvs[t // 16, :, :, t % 16] = sm.vs[:, :, t]
    return pk, pv, pks, pvs, ident


@pytest.fixture(scope="module")
def eng_mod(torch_dev):
    from tenzo_amd import engine
    return engine


# six chained steps as for int8_fused (each step's last-bit attention differences
# can move an activation code by one, ~1e-3 of the logits, so longer chains are
# not held to 1e-3); context 14 crosses into a new block at the third step
@pytest.mark.parametrize("mode,ctx", [("graph", 9), ("eager", 14), ("graph", 600), ("graph", 14),
                                      ("persistent", 0), ("persistent", 14),
                                      ("persistent", 600), ("persistent", 2039)])
def test_engine_paged_matches_oracle(eng_mod, mode, ctx):
    """Graph, eager and persistent (one launch per token: statistics of every
    chunk of a kv head combined in-kernel before the values) engines against
    the oracle's paged step; the persistent cases cover one chunk (first
    token), short chunks and 8-token chunks spread over 128 blocks."""
    cfg = CFG if ctx < 1000 else synth.DecodeConfig(**{**CFG.__dict__, "max_seq": 2048})
    sm = synth.make_model(cfg, seed=71, ctx=ctx)
    om = oracle.OracleModel(sm, kv_mode=3, kv=to_pools(sm, cfg))
    with eng_mod.Engine(cfg, kv_mode="paged_int8") as e:
        e.set_model(sm)
        e.set_mode(mode)
        assert e.mode == mode
        tok = 5
        for i in range(6):
            print(f"step {i} mode={mode} ctx={ctx}", flush=True)
            got = e.step(tok)
            ref_tok, ref_logits, ref_hidden = om.step(tok, ctx + i, CFG.theta)
            assert rel(e.buffer("x"), ref_hidden) < 1e-3
            assert rel(e.logits(), ref_logits) < 1e-3
            assert got == ref_tok
            tok = got
        n = ctx + 6
        np.testing.assert_array_equal(e.block_table(), np.arange((n + 15) // 16))
        kc, vc, ks, vs = e.get_kv(n)
        np.testing.assert_array_equal(kc[:, :, :ctx], sm.kc[:, :, :ctx])
        for t in range(ctx, n):
            for g, r in ((kc, om.kc), (vc, om.vc)):
                new_g, new_r = g[:, :, t].astype(int), r[t // 16, :, :, t % 16].astype(int)
                assert (new_g != new_r).mean() < 0.01 and np.abs(new_g - new_r).max() <= 1


def test_engine_paged_reference_goldens(eng_mod):
    """The compiled reference engine's greedy steps with kv_mode paged_int8
    (decode_paged fixture: 18 steps from an empty cache, over two blocks)."""
    z = np.load(os.path.join(GOLD, "decode_paged.npz"))
    sm = load_tiny_model(np.load(os.path.join(GOLD, "decode_tiny.npz")))
    cfg = synth.DecodeConfig(**{**TINY.__dict__, "max_seq": int(z["max_seq"])})
    sm.cfg = cfg
    sm.ctx = 0
    with eng_mod.Engine(cfg, kv_mode="paged_int8") as e:
        e.set_model(sm)
        for i, t in enumerate(z["tokens"]):
            tok = e.step(int(t))
            assert rel(e.buffer("x"), z["hidden"][i]) < 1e-3
            assert rel(e.logits(), z["logits"][i]) < 1e-3
            assert tok == z["out_tokens"][i]
        np.testing.assert_array_equal(e.block_table(), z["block_table"])
        n = len(z["tokens"])
        kc, vc, ks, vs = e.get_kv(n)
        bt = z["block_table"]
        for t in range(n):
            g, r = kc[:, :, t].astype(int), z["pk"][bt[t // 16], :, :, t % 16].astype(int)
            assert (g != r).mean() < 0.01 and np.abs(g - r).max() <= 1
        e.reset()
        assert e.seq_len == 0 and len(e.block_table()) == 0


@pytest.mark.parametrize("kv_mode", ["paged_int8", "tl1_fused", "popcount_fused"])
def test_engine_kv_modes_chained_decode_and_prefill(eng_mod, kv_mode):
    """Chained decode on the device (tenzo_hip_engine_decode) equals one step
    at a time, and the batched prefill entry point equals tenzo_prefill_token
    per token, across a block boundary; reset frees the sequence."""
    sm = synth.make_model(CFG, seed=73, ctx=0)
    toks = [3, 77, 1000, 5, 42, 9, 600, 11, 12, 13, 14, 15, 16, 17]
    with eng_mod.Engine(CFG, kv_mode=kv_mode) as a, eng_mod.Engine(CFG, kv_mode=kv_mode) as b:
        for e in (a, b):
            e.set_model(sm)
            e.set_mode("graph")  # the batched prefill's own arithmetic (not the persistent kernel's)
        a.prefill_batch(toks)
        for t in toks:
            b.prefill(t)
        assert a.seq_len == b.seq_len == len(toks)
        got, _ = a.decode(7, 6)
        ref = []
        tok = 7
        for _ in range(6):
            tok = b.step(tok)
            ref.append(tok)
        assert list(got) == ref
        np.testing.assert_array_equal(a.logits(), b.logits())
        n = len(toks) + 6
        for x, y in zip(a.get_kv(n), b.get_kv(n)):
            np.testing.assert_array_equal(x, y)
        if kv_mode == "paged_int8":
            np.testing.assert_array_equal(a.block_table(), np.arange(2))
            a.reset()
            assert len(a.block_table()) == 0
            a.prefill_batch(toks[:3])
            np.testing.assert_array_equal(a.block_table(), [0])


def test_engine_paged_kv_round_trip(eng_mod, torch_dev):
    """set_kv / get_kv move every (layer, kv head) row through the block table in one
    staging pass: 30 layers x 5 kv heads at a ragged length (1000 tokens, a partial last
    block) from host buffers, then a shorter cache (333 tokens) from device buffers,
    read back bit for bit."""
    torch = torch_dev
    cfg = synth.DecodeConfig(hidden=640, n_q_heads=5, n_kv_heads=5, n_layers=30, ffn=64,
                             vocab=256, max_seq=1024)
    rng = np.random.default_rng(5)
    n = 1000
    shape = (cfg.n_layers, cfg.n_kv_heads, n)
    kc = rng.integers(-128, 128, shape + (128,), dtype=np.int8)
    vc = rng.integers(-128, 128, shape + (128,), dtype=np.int8)
    ks = rng.random(shape, dtype=np.float32)
    vs = rng.random(shape, dtype=np.float32)
    with eng_mod.Engine(cfg, kv_mode="paged_int8") as e:
        print("paged set_kv host n=1000", flush=True)
        e.set_kv(kc, vc, ks, vs, n)
        assert e.seq_len == n
        np.testing.assert_array_equal(e.block_table(), np.arange((n + 15) // 16))
        for got, want in zip(e.get_kv(n), (kc, vc, ks, vs)):
            np.testing.assert_array_equal(got, want)
        m = 333
        src = [np.ascontiguousarray(a[:, :, ::-1][:, :, :m]) for a in (kc, vc, ks, vs)]
        dev = [torch.from_numpy(a).cuda() for a in src]
        print("paged set_kv device n=333", flush=True)
        e.set_kv_device(*(t.data_ptr() for t in dev), m)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(e.block_table(), np.arange((m + 15) // 16))
        for got, want in zip(e.get_kv(m), src):
            np.testing.assert_array_equal(got, want)
