"""The persistent decode kernel at exactly the benchmarked configuration
(the BitNet-b1.58-2B shape - 30 layers, hidden 2560, FFN
6912, 20 query / 5 KV heads of 128, vocabulary 128256, an INT8 KV cache with
fp16 scales prefilled with 4096 tokens, RoPE theta 500000), with the model
built by bench.py's own builder, against the CPU oracle:

* layer by layer, teacher-forced: every stage is recomputed on the CPU from
  the engine's own input to that stage (forward_layer_raw,
  TenzoEngine.cpp:1522-1632). The int32 TL1 sums of q|k|v, out, gate|up and
  down, the residual vectors h1 and x and the appended KV codes and scales are
  bit-exact; the attention output is within 1e-5 (the same fp32 terms, the
  softmax sums grouped by context chunk);
* the LM head from the engine's final hidden state (compute_logits :1634-1720):
  logits bit-exact, greedy token equal;
* end to end against the oracle's own chain from the embedding: greedy token
  equal, hidden state and logits within 1e-3, and the number of activation
  codes that differ between the two chains (a code can only differ where an
  attention value decided by a last-bit difference sits on a rounding tie) is
  printed and held below 0.1%;
* the chained decode the benchmark times (tenzo_hip_engine_decode) for 1..4
  steps: each step stage by stage from the engine's own state, the chain equal
  to the per-step API, and the oracle's own chain alongside (step 1 asserted,
  later steps reported: see test_full_shape_chained_decode).

This is the split and chunk layout the benchmark runs: QKV in 4 K-slices, O
and down in 6, gate|up in 1, 51 attention chunks of 81 tokens per kv head and
2004 LM-head row blocks over 256 workgroups."""
import numpy as np
import pytest

import oracle
from tenzo_amd import synth

pytestmark = pytest.mark.gpu

CTX = 4096


def rel(a, b):
    return np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30)


@pytest.fixture(scope="module")
def full():
    import torch
    assert torch.cuda.is_available(), "GPU test needs a visible GPU"
    import bench
    cfg = synth.BITNET_2B
    print("building the BitNet-2B-shaped model (bench.build_model)", flush=True)
    e, host = bench.build_model(torch, cfg, CTX)
    assert e.mode == "persistent"
    L, Hkv, S = cfg.n_layers, cfg.n_kv_heads, cfg.max_seq
    layers = []
    for tl1, scale, norms in host["layers"]:
        layers.append(synth.LayerWeights({p: t.cpu().numpy() for p, t in tl1.items()},
                                         dict(scale), norms["in_norm"], norms["attn_sub_norm"],
                                         norms["post_norm"], norms["ffn_sub_norm"]))
    kc = np.zeros((L, Hkv, S, 128), np.int8)
    vc = np.zeros_like(kc)
    ks = np.zeros((L, Hkv, S), np.float32)
    vs = np.zeros_like(ks)
    kc[:, :, :CTX] = host["kc"].cpu().numpy()
    vc[:, :, :CTX] = host["vc"].cpu().numpy()
    ks[:, :, :CTX] = host["ks"].float().cpu().numpy()
    vs[:, :, :CTX] = host["vs"].float().cpu().numpy()
    sm = synth.SynthModel(cfg, layers, host["final_norm"], host["head"].cpu().numpy(),
                          host["hs"].cpu().numpy(), kc, vc, ks, vs, CTX)
    del host
    tok_in = 1234
    print("engine step at position 4096", flush=True)
    tok = e.step(tok_in)
    yield e, sm, tok_in, tok
    e.close()


def lin_acc(w, inp, N, K):
    """(int32 sums sum_k (w+1) a_k as the engine keeps them, codes, 1/scale)."""
    codes, inv = oracle.quant31(inp)
    acc = oracle.tl1_gemv_i32(w, codes, N, K)
    return acc + np.int32(codes.astype(np.int64).sum()), codes, inv


def y_of(acc_u, codes, inv, scale):
    """GEMV output from the engine's sums: float(acc - code_sum) * (inv * scale)."""
    a = (acc_u - np.int32(codes.astype(np.int64).sum())).astype(np.float32)
    return a * np.float32(np.float32(inv) * np.float32(scale))


def check_step_teacher_forced(e, sm, tok, pos, kc, vc, ks, vs, label=""):
    """The engine's last step (token tok at position pos) stage by stage: every
    stage is recomputed on the CPU from the engine's own input to that stage
    over the KV cache arrays given (rows 0..pos-1, the oracle's row for pos is
    appended into them). Integer stages and the vectors built from them are
    bit-exact, attention within 1e-5; then the appended KV rows, the logits
    from the engine's final hidden state and the greedy token. Returns the
    token."""
    cfg = sm.cfg
    H, F, qd, kvd = cfg.hidden, cfg.ffn, cfg.q_dim, cfg.kv_dim
    cs = oracle.rope_table(cfg.theta, pos)
    x0 = np.empty(H, np.float32)
    oracle.lib().orc_embed_i8(oracle._ptr(sm.embed), oracle._ptr(sm.embed_scales), H, tok,
                              oracle._ptr(x0))
    for l in range(cfg.n_layers):
        where = f"{label}layer {l}"
        lw = sm.layers[l]
        x = e.layer_state(l, "x")
        if l == 0:
            np.testing.assert_array_equal(x, x0, err_msg=f"{where} embedding")
        # Q|K|V from the layer input
        xn = oracle.rms_norm(x, lw.in_norm)
        acc = e.layer_state(l, "acc_qkv")
        outs = []
        for name, rows, off in (("q", qd, 0), ("k", kvd, qd), ("v", kvd, qd + kvd)):
            a, codes, inv = lin_acc(lw.tl1[name], xn, rows, H)
            np.testing.assert_array_equal(acc[off:off + rows], a, err_msg=f"{where} {name}")
            outs.append(y_of(a, codes, inv, lw.scale[name]))
        q, k, v = outs
        # attention over the cache given and the new token
        attn, _, _ = oracle.attention_step(q, k, v, kc[l], vc[l], ks[l], vs[l], cfg.n_q_heads,
                                           cfg.n_kv_heads, cfg.max_seq, pos, cs, f16_scales=True)
        got_attn = e.layer_state(l, "attn_out")
        assert rel(got_attn, attn) < 1e-5, f"{where} attention"
        # out projection and residual from the engine's attention output
        a, codes, inv = lin_acc(lw.tl1["o"], oracle.rms_norm(got_attn, lw.attn_sub_norm), H, qd)
        np.testing.assert_array_equal(e.layer_state(l, "acc_o"), a, err_msg=f"{where} o")
        h1 = (x + y_of(a, codes, inv, lw.scale["o"])).astype(np.float32)
        np.testing.assert_array_equal(e.layer_state(l, "h1"), h1, err_msg=f"{where} h1")
        # gate|up
        pn = oracle.rms_norm(h1, lw.post_norm)
        acc = e.layer_state(l, "acc_gu")
        a_g, c_g, i_g = lin_acc(lw.tl1["gate"], pn, F, H)
        a_u, c_u, i_u = lin_acc(lw.tl1["up"], pn, F, H)
        np.testing.assert_array_equal(acc[:F], a_g, err_msg=f"{where} gate")
        np.testing.assert_array_equal(acc[F:], a_u, err_msg=f"{where} up")
        g, u = y_of(a_g, c_g, i_g, lw.scale["gate"]), y_of(a_u, c_u, i_u, lw.scale["up"])
        r = np.maximum(g, np.float32(0))
        act = ((r * r) * u).astype(np.float32)
        # down and the residual
        a, codes, inv = lin_acc(lw.tl1["down"], oracle.rms_norm(act, lw.ffn_sub_norm), H, F)
        np.testing.assert_array_equal(e.layer_state(l, "acc_down"), a, err_msg=f"{where} down")
        x_next = (h1 + y_of(a, codes, inv, lw.scale["down"])).astype(np.float32)
        nxt = e.layer_state(l + 1, "x") if l + 1 < cfg.n_layers else e.buffer("x")
        np.testing.assert_array_equal(nxt, x_next, err_msg=f"{where} output")
    # the appended KV codes and scales of every layer
    gk, gv, gks, gvs = e.get_kv(pos + 1)
    np.testing.assert_array_equal(gk[:, :, pos], kc[:, :, pos])
    np.testing.assert_array_equal(gv[:, :, pos], vc[:, :, pos])
    np.testing.assert_array_equal(gks[:, :, pos], ks[:, :, pos])
    np.testing.assert_array_equal(gvs[:, :, pos], vs[:, :, pos])
    # LM head from the engine's final hidden state: bit-exact logits
    xf = e.buffer("x")
    lg, _, _ = oracle.lm_head(oracle.rms_norm(xf, sm.final_norm), sm.embed, sm.embed_scales)
    np.testing.assert_array_equal(e.logits(), lg)
    return oracle.argmax(lg)


def test_full_shape_layers_teacher_forced(full):
    e, sm, tok_in, tok = full
    assert check_step_teacher_forced(e, sm, tok_in, CTX, sm.kc, sm.vc, sm.ks, sm.vs) == tok


def oracle_step(sm, tok, pos, kc, vc, ks, vs, e=None):
    """One step of the oracle's own chain: token tok at position pos over its own KV cache
    arrays (the new K/V rows appended into them). With an engine, the activation codes of
    every GEMV input are also formed from the engine's inputs to that stage (its last
    step's layer state) and the codes that differ are counted. Returns the final hidden
    state, the logits and (differing codes, codes compared)."""
    cfg = sm.cfg
    H, F, qd, kvd = cfg.hidden, cfg.ffn, cfg.q_dim, cfg.kv_dim
    cs = oracle.rope_table(cfg.theta, pos)
    x = np.empty(H, np.float32)
    oracle.lib().orc_embed_i8(oracle._ptr(sm.embed), oracle._ptr(sm.embed_scales), H, tok,
                              oracle._ptr(x))
    flips, total = 0, 0

    def stage(w, inp, N, K, scale, eng_inp):
        nonlocal flips, total
        codes, inv = oracle.quant31(inp)
        if eng_inp is not None:
            eng_codes, _ = oracle.quant31(eng_inp)
            flips += int((codes != eng_codes).sum())
            total += codes.size
        acc = oracle.tl1_gemv_i32(w, codes, N, K)
        return acc.astype(np.float32) * np.float32(np.float32(inv) * np.float32(scale))

    def eng_norm(l, name, w):
        return None if e is None else oracle.rms_norm(e.layer_state(l, name), w)

    for l in range(cfg.n_layers):
        lw = sm.layers[l]
        xn = oracle.rms_norm(x, lw.in_norm)
        exn = eng_norm(l, "x", lw.in_norm)
        q = stage(lw.tl1["q"], xn, qd, H, lw.scale["q"], exn)
        k = stage(lw.tl1["k"], xn, kvd, H, lw.scale["k"], exn)
        v = stage(lw.tl1["v"], xn, kvd, H, lw.scale["v"], exn)
        attn, _, _ = oracle.attention_step(q, k, v, kc[l], vc[l], ks[l], vs[l], cfg.n_q_heads,
                                           cfg.n_kv_heads, cfg.max_seq, pos, cs, f16_scales=True)
        h1 = (x + stage(lw.tl1["o"], oracle.rms_norm(attn, lw.attn_sub_norm), H, qd,
                        lw.scale["o"], eng_norm(l, "attn_out", lw.attn_sub_norm))).astype(np.float32)
        pn = oracle.rms_norm(h1, lw.post_norm)
        epn = eng_norm(l, "h1", lw.post_norm)
        g = stage(lw.tl1["gate"], pn, F, H, lw.scale["gate"], epn)
        u = stage(lw.tl1["up"], pn, F, H, lw.scale["up"], epn)
        r = np.maximum(g, np.float32(0))
        act = ((r * r) * u).astype(np.float32)
        edn = None
        if e is not None:
            # the engine's act from its own gate|up sums (codes of its GU input)
            ec, einv = oracle.quant31(epn)
            eacc = e.layer_state(l, "acc_gu")
            eg = y_of(eacc[:F], ec, einv, lw.scale["gate"])
            eu = y_of(eacc[F:], ec, einv, lw.scale["up"])
            er = np.maximum(eg, np.float32(0))
            edn = oracle.rms_norm(((er * er) * eu).astype(np.float32), lw.ffn_sub_norm)
        x = (h1 + stage(lw.tl1["down"], oracle.rms_norm(act, lw.ffn_sub_norm), H, F,
                        lw.scale["down"], edn)).astype(np.float32)
    lg, _, _ = oracle.lm_head(oracle.rms_norm(x, sm.final_norm), sm.embed, sm.embed_scales)
    return x, lg, (flips, total)


def own_cache(sm):
    """Copies of the prefilled KV cache for an oracle chain (nothing past CTX)."""
    kc, vc = sm.kc.copy(), sm.vc.copy()
    ks, vs = sm.ks.copy(), sm.vs.copy()
    for a in (kc, vc, ks, vs):
        a[:, :, CTX:] = 0
    return kc, vc, ks, vs


def test_full_shape_end_to_end(full):
    """The oracle's own chain from the embedding (its attention summed in
    sequence order) against the engine's step."""
    e, sm, tok_in, tok = full
    x, lg, (flips, total) = oracle_step(sm, tok_in, CTX, *own_cache(sm), e)
    print(f"end to end: hidden rel {rel(e.buffer('x'), x):.2e}, logits rel "
          f"{rel(e.logits(), lg):.2e}, activation codes differing {flips} of {total}",
          flush=True)
    assert rel(e.buffer("x"), x) < 1e-3
    assert rel(e.logits(), lg) < 1e-3
    assert tok == oracle.argmax(lg)
    assert flips <= total * 1e-3


N_CHAIN = 4


def test_full_shape_chained_decode(full):
    """tenzo_hip_engine_decode, the call bench.py times (each greedy token fed
    to the next step on the device, the position read from device memory), at
    the benchmarked shape from position 4096, for n = 1..N_CHAIN chained steps
    from the same start:

    * the chain's n-th step, stage by stage against the oracle given the
      engine's own state (its token, the KV rows its earlier steps appended):
      integer stages, residual vectors, appended KV rows and logits bit-exact,
      attention within 1e-5, and its token the argmax of its logits;
    * the chain equals the per-step API (tenzo_hip_engine_generate_step per
      token): same tokens, bit-identical hidden state and logits;
    * the oracle's own chain (its tokens, its KV rows) alongside: step 1 must
      give the same token with hidden state and logits within 1e-3 and no
      activation code differing. Later steps are printed, not asserted: in
      this random-weight model a last-bit difference is not damped - the fp32
      attention sums of step 1 (another order than the oracle's) move the
      layers' float scales by an ulp, a few of the KV codes step 1 appends
      flip by 1 at rounding ties (counted and printed here), and from step 2
      on the two chains' states separate."""
    e, sm, tok_in, _ = full
    cfg = sm.cfg
    okc, ovc, oks, ovs = own_cache(sm)
    otok = tok_in
    for n in range(1, N_CHAIN + 1):
        e.rewind(CTX)
        toks, _ = e.decode(tok_in, n)
        toks = [int(t) for t in toks]
        pos = CTX + n - 1
        xc, lc = e.buffer("x"), e.logits()
        # stage by stage from the engine's own state: its KV rows before pos
        gk, gv, gks, gvs = e.get_kv(pos)
        kc = np.zeros_like(sm.kc)
        vc, ks, vs = np.zeros_like(sm.vc), np.zeros_like(sm.ks), np.zeros_like(sm.vs)
        kc[:, :, :pos], vc[:, :, :pos] = gk, gv
        ks[:, :, :pos], vs[:, :, :pos] = gks, gvs
        step_in = tok_in if n == 1 else toks[n - 2]
        assert check_step_teacher_forced(e, sm, step_in, pos, kc, vc, ks, vs,
                                         f"chained step {n}: ") == toks[-1]
        # the per-step API from the same start
        e.rewind(CTX)
        t, steps = tok_in, []
        for _ in range(n):
            t = e.step(t)
            steps.append(t)
        assert steps == toks
        np.testing.assert_array_equal(e.buffer("x"), xc)
        np.testing.assert_array_equal(e.logits(), lc)
        # the oracle's own chain
        ox, olg, (flips, total) = oracle_step(sm, otok, pos, okc, ovc, oks, ovs, e)
        otok = oracle.argmax(olg)
        kv_flips = (int((gk[:, :, CTX:] != okc[:, :, CTX:pos]).sum()) +
                    int((gv[:, :, CTX:] != ovc[:, :, CTX:pos]).sum()))
        hx, hl = rel(xc, ox), rel(lc, olg)
        print(f"chained step {n} (position {pos}): engine token {toks[-1]}, oracle chain token "
              f"{otok}; against the oracle chain: hidden rel {hx:.2e}, logits rel {hl:.2e}, "
              f"activation codes differing {flips} of {total}, KV codes of earlier chained "
              f"steps differing {kv_flips}", flush=True)
        if n == 1:
            assert toks[-1] == otok and hx < 1e-3 and hl < 1e-3 and flips == 0
