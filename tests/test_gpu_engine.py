"""The engine (include/tenzo.h on the GPU) against the CPU oracle's decode step
and the compiled reference's whole-engine goldens.

Bars: every integer stage (activation codes, TL1 int32 sums, KV codes) is
bit-exact given identical inputs; attention is an fp32 reduction in another
order (1e-3), so chained steps are compared at 1e-3 on the hidden state and
logits, and the greedy tokens must agree."""
import os

import numpy as np
import pytest

import oracle
from tenzo_amd import synth
from tests.golden.make_golden import TINY, load_tiny_model

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def eng_mod():
    import torch
    assert torch.cuda.is_available(), "GPU test needs a visible GPU"
    from tenzo_amd import engine
    return engine


def rel(a, b):
    return np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30)


CFG = synth.DecodeConfig(hidden=512, n_q_heads=4, n_kv_heads=1, n_layers=3, ffn=1024,
                         vocab=2048, max_seq=64, theta=10000.0)


@pytest.mark.parametrize("mode", ["persistent", "graph", "eager"])
def test_engine_steps_match_oracle(eng_mod, mode):
    sm = synth.make_model(CFG, seed=41, ctx=9)
    om = oracle.OracleModel(sm, f16_kv_scales=True)
    with eng_mod.Engine(CFG) as e:
        e.set_model(sm)
        e.set_mode(mode)
        assert e.mode == mode
        assert e.seq_len == 9
        tok = 5
        for i in range(6):
            print(f"step {i} mode={mode}", flush=True)
            got = e.step(tok)
            ref_tok, ref_logits, ref_hidden = om.step(tok, sm.ctx + i, CFG.theta)
            assert rel(e.buffer("x"), ref_hidden) < 1e-3
            assert rel(e.logits(), ref_logits) < 1e-3
            assert got == ref_tok
            tok = got
        assert e.seq_len == 15
        # appended KV codes agree except for rare rounding-tie flips of +-1
        kc, vc, ks, vs = e.get_kv(15)
        for g, r in ((kc, om.kc), (vc, om.vc)):
            new_g, new_r = g[:, :, 9:15].astype(int), r[:, :, 9:15].astype(int)
            assert (new_g != new_r).mean() < 0.01 and np.abs(new_g - new_r).max() <= 1
        np.testing.assert_array_equal(kc[:, :, :9], sm.kc[:, :, :9])


@pytest.mark.parametrize("hidden,Hq,Hkv,ctx", [(512, 4, 4, 30), (512, 4, 2, 300), (1024, 8, 1, 700),
                                               (1024, 8, 8, 4000), (512, 4, 1, 1)])
def test_persistent_head_layouts_and_context(eng_mod, hidden, Hq, Hkv, ctx):
    """Persistent kernel for every GQA group size (1, 2, 4, 8), a context whose
    chunks are longer than the preloaded rounds (8 kv heads at 4000), and a
    first token (context 1)."""
    cfg = synth.DecodeConfig(hidden=hidden, n_q_heads=Hq, n_kv_heads=Hkv, n_layers=2, ffn=768,
                             vocab=1000, max_seq=ctx + 4, theta=10000.0)
    print(f"persistent H={hidden} Hq={Hq} Hkv={Hkv} ctx={ctx}", flush=True)
    sm = synth.make_model(cfg, seed=ctx + Hkv, ctx=ctx - 1)
    om = oracle.OracleModel(sm, f16_kv_scales=True)
    with eng_mod.Engine(cfg) as e:
        e.set_model(sm)
        assert e.mode == "persistent"
        tok = 17
        for i in range(3):
            got = e.step(tok)
            ref_tok, ref_logits, ref_hidden = om.step(tok, sm.ctx + i, cfg.theta)
            assert rel(e.buffer("x"), ref_hidden) < 1e-3
            assert rel(e.logits(), ref_logits) < 1e-3
            assert got == ref_tok
            tok = got


def test_persistent_more_chunks_than_workgroups(eng_mod):
    """4 kv heads x 67 chunks of 256 tokens at context 17000: more attention
    tasks than workgroups, so workgroups run several chunks and one merger per
    kv head combines them. Checked where the attention is exact up to its
    summation order: the last layer's output against the oracle's attention on
    the engine's own q and cache (1e-5), and every step against graph mode.
    (End to end against the oracle this context is fragile: one +-31
    activation code at a rounding tie, decided by a 1e-6 difference in an
    attention sum, moves the hidden state by ~1e-2.)"""
    cfg = synth.DecodeConfig(hidden=1024, n_q_heads=8, n_kv_heads=4, n_layers=2, ffn=768,
                             vocab=1000, max_seq=17004, theta=10000.0)
    ctx = 17000
    sm = synth.make_model(cfg, seed=ctx + 4, ctx=ctx - 1)
    outs = {}
    for mode in ("persistent", "graph"):
        with eng_mod.Engine(cfg) as e:
            e.set_model(sm)
            e.set_mode(mode)
            tok, seq = 17, []
            for i in range(3):
                print(f"{mode} step {i}", flush=True)
                tok = e.step(tok)
                n = ctx + i
                kc, vc, ks, vs = e.get_kv(n)
                q = e.buffer("qkv")[:cfg.q_dim].copy()
                qr = oracle.rope_apply(q, oracle.rope_table(cfg.theta, n - 1))
                ref = oracle.attn_int8(qr, kc[1], vc[1], ks[1], vs[1], 8, 4, n, n)
                assert rel(e.buffer("attn_out"), ref) < 1e-5
                seq.append((tok, e.logits(), e.buffer("x")))
            outs[mode] = seq
    for (tp, lp, xp), (tg, lg, xg) in zip(outs["persistent"], outs["graph"]):
        assert tp == tg
        assert rel(xp, xg) < 1e-5 and rel(lp, lg) < 1e-5


def test_modes_agree(eng_mod):
    """Persistent, graph and eager steps of one model: integer stages equal,
    fp32 outputs equal up to the attention reduction order."""
    sm = synth.make_model(CFG, seed=53, ctx=20)
    outs = {}
    for mode in ("persistent", "graph", "eager"):
        with eng_mod.Engine(CFG) as e:
            e.set_model(sm)
            e.set_mode(mode)
            toks = [e.step(t) for t in (3, 1, 4, 1, 5)]
            outs[mode] = (toks, e.logits(), e.buffer("x"), e.get_kv(25))
    p, g, z = outs["persistent"], outs["graph"], outs["eager"]
    assert p[0] == g[0] == z[0]
    np.testing.assert_array_equal(g[1], z[1])  # same kernels, same chunking
    assert rel(p[1], g[1]) < 1e-5 and rel(p[2], g[2]) < 1e-5
    for a, b in zip(p[3], g[3]):
        assert (np.asarray(a) != np.asarray(b)).mean() < 0.01


@pytest.mark.parametrize("mode", ["persistent", "graph", "eager"])
def test_chained_decode_equals_steps(eng_mod, mode):
    """tenzo_hip_engine_decode (tokens fed back on the device) produces the
    same tokens, logits and cache as one generate_step per token."""
    sm = synth.make_model(CFG, seed=57, ctx=11)
    with eng_mod.Engine(CFG) as a, eng_mod.Engine(CFG) as b:
        a.set_model(sm)
        b.set_model(sm)
        a.set_mode(mode)
        b.set_mode(mode)
        toks, ms = a.decode(7, 9)
        assert ms > 0 and a.seq_len == 20
        ref, t = [], 7
        for _ in range(9):
            t = b.step(t)
            ref.append(t)
        assert list(toks) == ref
        np.testing.assert_array_equal(a.logits(), b.logits())
        for x, y in zip(a.get_kv(20), b.get_kv(20)):
            np.testing.assert_array_equal(x, y)
        # the next step continues from the chained state
        assert a.step(int(toks[-1])) == b.step(ref[-1])


def test_persistent_abort_is_reported(eng_mod, monkeypatch):
    """Failure handling, forced from the host: with an in-kernel poll budget of
    zero the first wait that finds its condition unmet gives up and every
    workgroup leaves the kernel at its next poll. TENZO_HIP_SPIN_LIMIT sets the
    budget under the ordinary launch and TENZO_HIP_SPIN_LIMIT_COOP under the
    cooperative one (both read when the engine is made).

    With both at zero, the step that aborted under the ordinary launch is
    rerun once under the cooperative launch, aborts again, and the call
    reports the timeout instead of a token -- in a chained decode and in a
    single step -- and the per-layer state is refused afterwards."""
    sm = synth.make_model(CFG, seed=61, ctx=11)
    monkeypatch.setenv("TENZO_HIP_SPIN_LIMIT", "0")
    monkeypatch.setenv("TENZO_HIP_SPIN_LIMIT_COOP", "0")
    a = eng_mod.Engine(CFG)
    monkeypatch.delenv("TENZO_HIP_SPIN_LIMIT")
    monkeypatch.delenv("TENZO_HIP_SPIN_LIMIT_COOP")
    with a:
        a.set_model(sm)
        a.set_mode("persistent")
        with pytest.raises(RuntimeError, match="timed out.*cooperative"):
            a.decode(7, 3)
        with pytest.raises(RuntimeError, match="last step did not run"):
            a.layer_state(0, "x")
        with pytest.raises(RuntimeError, match="timed out"):
            a.step(7)


def test_persistent_abort_recovers(eng_mod, monkeypatch):
    """An abort under the ordinary launch (its poll budget forced to zero) is
    recovered within the call: the step that aborted -- and, in a chained
    decode, every step after it, which returned at entry -- is rerun under
    the cooperative launch (full budget), so the reference API still returns
    the token. Tokens equal the oracle's greedy chain, and the hidden state
    after the recovered steps equals the oracle's to 1e-3."""
    sm = synth.make_model(CFG, seed=61, ctx=11)
    om = oracle.OracleModel(sm, f16_kv_scales=True)
    ref, t = [], 7
    for i in range(5):
        t, _, hidden = om.step(t, sm.ctx + i, CFG.theta)
        ref.append(t)
    monkeypatch.setenv("TENZO_HIP_SPIN_LIMIT", "0")
    a = eng_mod.Engine(CFG)
    b = eng_mod.Engine(CFG)
    monkeypatch.delenv("TENZO_HIP_SPIN_LIMIT")
    with a, b:
        a.set_model(sm)
        b.set_model(sm)
        a.set_mode("persistent")
        b.set_mode("persistent")
        toks, _ = a.decode(7, 3)
        assert list(toks) == ref[:3]
        toks2, _ = a.decode(int(toks[-1]), 2)  # (now on the cooperative launch)
        assert list(toks2) == ref[3:]
        assert rel(a.buffer("x"), hidden) < 1e-3
        assert b.step(7) == ref[0]
        assert b.step(ref[0]) == ref[1]


def test_engine_first_layer_stages_bit_exact(eng_mod):
    """One layer, stage by stage from the engine's own buffers: QKV from the
    embedded token, O/residual, gate|up and down/residual are bit-exact."""
    cfg = synth.DecodeConfig(hidden=512, n_q_heads=4, n_kv_heads=2, n_layers=1, ffn=1024,
                             vocab=512, max_seq=32, theta=10000.0)
    sm = synth.make_model(cfg, seed=43, ctx=4)
    lw = sm.layers[0]
    with eng_mod.Engine(cfg) as e:
        e.set_model(sm)
        e.step(77)
        x0 = sm.embed[77].astype(np.float32) * sm.embed_scales[77]

        def lin(name, inp, N, K):
            codes, inv = oracle.quant31(inp)
            acc = oracle.tl1_gemv_i32(lw.tl1[name], codes, N, K)
            return acc.astype(np.float32) * np.float32(inv * lw.scale[name])

        H, F = cfg.hidden, cfg.ffn
        xn = oracle.rms_norm(x0, lw.in_norm)
        qkv = np.concatenate([lin("q", xn, cfg.q_dim, H), lin("k", xn, cfg.kv_dim, H),
                              lin("v", xn, cfg.kv_dim, H)])
        np.testing.assert_array_equal(e.buffer("qkv"), qkv)
        attn = e.buffer("attn_out")
        h1 = (x0 + lin("o", oracle.rms_norm(attn, lw.attn_sub_norm), H, H)).astype(np.float32)
        np.testing.assert_array_equal(e.buffer("h1"), h1)
        pn = oracle.rms_norm(h1, lw.post_norm)
        gu = np.concatenate([lin("gate", pn, F, H), lin("up", pn, F, H)])
        np.testing.assert_array_equal(e.buffer("gate_up"), gu)
        g, u = gu[:F], gu[F:]
        act = (np.maximum(g, np.float32(0)) ** 2 * u).astype(np.float32)
        x1 = (h1 + lin("down", oracle.rms_norm(act, lw.ffn_sub_norm), H, F)).astype(np.float32)
        np.testing.assert_array_equal(e.buffer("x"), x1)
        # attention of this step against the oracle from the same q/k/v
        kc, vc = sm.kc[0].copy(), sm.vc[0].copy()
        ks, vs = sm.ks[0].copy(), sm.vs[0].copy()
        out, _, _ = oracle.attention_step(qkv[:cfg.q_dim], qkv[cfg.q_dim:cfg.q_dim + cfg.kv_dim],
                                          qkv[cfg.q_dim + cfg.kv_dim:], kc, vc, ks, vs,
                                          cfg.n_q_heads, cfg.n_kv_heads, cfg.max_seq, 4,
                                          oracle.rope_table(cfg.theta, 4), f16_scales=True)
        assert rel(attn, out) < 1e-5


def test_engine_against_reference_goldens(eng_mod):
    """The compiled reference engine's own greedy steps (decode_tiny fixture)."""
    z = np.load(os.path.join(GOLD, "decode_tiny.npz"))
    sm = load_tiny_model(z)
    with eng_mod.Engine(TINY) as e:
        e.set_model(sm)
        for i, t in enumerate(z["tokens"]):
            tok = e.step(int(t))
            assert rel(e.buffer("x"), z["hidden"][i]) < 1e-3
            assert rel(e.logits(), z["logits"][i]) < 1e-3
            assert tok == z["out_tokens"][i]


def test_engine_prefill_then_decode_equals_steps(eng_mod):
    sm = synth.make_model(CFG, seed=45, ctx=0)
    toks = [3, 9, 27, 81, 243]
    with eng_mod.Engine(CFG) as a, eng_mod.Engine(CFG) as b:
        a.set_model(sm)
        b.set_model(sm)
        for t in toks[:-1]:
            a.prefill(t)
            b.step(t)
        assert a.seq_len == b.seq_len == len(toks) - 1
        assert a.step(toks[-1]) == b.step(toks[-1])
        np.testing.assert_array_equal(a.logits(), b.logits())
        a.reset()
        assert a.seq_len == 0


def test_engine_repetition_penalty(eng_mod):
    """The penalty of sample_top_k_top_p (:1735-1743) as the reference build
    evaluates it (oracle.rep_penalty, pinned to the compiled reference):
    repeated tokens compound, both signs of logit, out-of-range tokens skipped."""
    sm = synth.make_model(CFG, seed=47, ctx=3)
    with eng_mod.Engine(CFG) as e:
        e.set_model(sm)
        e.step(11)
        base = e.logits()
        order = np.argsort(base)
        for pen, past in ((1.3, [int(order[-1])] * 2 + [4]),
                          (0.7, [int(order[0]), int(order[-1]), int(order[-2]), int(order[-2])]),
                          (1.15, list(order[-40:]) + list(order[:40]) + [-3, CFG.vocab + 2])):
            e.reset()
            e.set_kv_from(sm)
            tok = e.step(11, penalty=pen, past=past)
            ref = oracle.rep_penalty(base, past, pen)
            np.testing.assert_array_equal(e.logits(), ref)
            assert tok == oracle.argmax(ref)


def test_engine_f32_lm_head(eng_mod):
    from tenzo_amd import _lib
    import ctypes
    cfg = synth.DecodeConfig(hidden=256, n_q_heads=2, n_kv_heads=1, n_layers=1, ffn=512,
                             vocab=300, max_seq=16, theta=10000.0)
    sm = synth.make_model(cfg, seed=49, ctx=2)
    E = np.random.default_rng(3).normal(0, 0.02, size=(cfg.vocab, cfg.hidden)).astype(np.float32)
    with eng_mod.Engine(cfg) as e:
        e.set_model(sm)
        L = _lib.load()
        assert L.tenzo_set_lm_head_f32(e.h, ctypes.c_void_p(E.ctypes.data), cfg.vocab,
                                       cfg.hidden) == 0
        tok = e.step(17)
        xn = oracle.rms_norm(e.buffer("x"), sm.final_norm)
        ref = E.astype(np.float64) @ xn.astype(np.float64)
        assert rel(e.logits(), ref) < 1e-5
        assert tok == int(np.argmax(e.logits()))


def test_engine_error_paths(eng_mod):
    from tenzo_amd import _lib
    import ctypes
    L = _lib.load()
    cfg = synth.DecodeConfig(hidden=256, n_q_heads=2, n_kv_heads=1, n_layers=1, ffn=512,
                             vocab=300, max_seq=4, theta=10000.0)
    sm = synth.make_model(cfg, seed=51, ctx=0)
    with eng_mod.Engine(cfg) as e:
        # no weights yet: the step is refused, not run
        p = eng_mod.SamplingParams(0.0, 0.9, 40, 1.0)
        assert L.tenzo_generate_step(e.h, 1, ctypes.byref(p), None, 0) == -1
        e.set_model(sm)
        assert L.tenzo_generate_step(e.h, cfg.vocab, ctypes.byref(p), None, 0) == -1  # bad token
        for t in range(4):
            e.step(t)
        assert L.tenzo_generate_step(e.h, 1, ctypes.byref(p), None, 0) == -1  # cache full
        assert b"full" in L.tenzo_hip_last_error()
        assert L.tenzo_set_layer_weights(None, 0, None) == -1
    bad = eng_mod.config_from(cfg)
    for mode in (b"fp32", b"int4_fused"):  # not provided on the GPU
        bad.kv_mode = mode
        assert not L.tenzo_create_engine(ctypes.byref(bad))
        assert b"kv_mode" in L.tenzo_hip_last_error()


@pytest.mark.parametrize("ffn", [1024, 8192])
def test_persistent_codes_at_rounding_ties(eng_mod, ffn):
    """Workgroups with GEMV tasks take their +-31 codes from an estimate of the
    RMS scale and recompute them with the exact one when an element lies
    within the estimate's error bound of a rounding tie. Here the embedding row
    of the token holds the values -62..62, each in many places, the first
    layer's input norm is 1, and so every odd value becomes z = 31 e / 62 = a
    half-integer: the exact path decides every one. The first layer's q|k|v
    sums, and every later stage, must still be bit-exact. ffn 8192 gives the
    gate|up stage 256 tasks, one per workgroup: then the workgroup of task 0
    computes the record itself."""
    cfg = synth.DecodeConfig(hidden=512, n_q_heads=4, n_kv_heads=1, n_layers=2, ffn=ffn,
                             vocab=1000, max_seq=16, theta=10000.0)
    sm = synth.make_model(cfg, seed=7, ctx=3)
    tok = 21
    sm.embed[tok] = (np.arange(cfg.hidden) % 125 - 62).astype(np.int8)
    sm.layers[0].in_norm[:] = 1.0
    print(f"persistent ties ffn={ffn}", flush=True)
    with eng_mod.Engine(cfg) as e:
        e.set_model(sm)
        assert e.mode == "persistent"
        e.step(tok)
        H, F, qd, kvd = cfg.hidden, cfg.ffn, cfg.q_dim, cfg.kv_dim
        x = e.layer_state(0, "x")
        y = oracle.rms_norm(x, sm.layers[0].in_norm)
        z = np.abs(y * (np.float32(31) / np.abs(y).max()))
        assert (np.abs(z - np.floor(z) - 0.5) < 1e-5).sum() > cfg.hidden // 3  # at ties
        for l in range(cfg.n_layers):
            lw = sm.layers[l]
            checks = (("acc_qkv", oracle.rms_norm(e.layer_state(l, "x"), lw.in_norm),
                       [("q", qd), ("k", kvd), ("v", kvd)], H),
                      ("acc_o", oracle.rms_norm(e.layer_state(l, "attn_out"), lw.attn_sub_norm),
                       [("o", H)], qd),
                      ("acc_gu", oracle.rms_norm(e.layer_state(l, "h1"), lw.post_norm),
                       [("gate", F), ("up", F)], H))
            for name, inp, mats, K in checks:
                c, _ = oracle.quant31(inp)
                acc, off = e.layer_state(l, name), 0
                for m, rows in mats:
                    ref = oracle.tl1_gemv_i32(lw.tl1[m], c, rows, K) + np.int32(c.astype(np.int64).sum())
                    np.testing.assert_array_equal(acc[off:off + rows], ref, err_msg=f"layer {l} {m}")
                    off += rows
