"""Writes tests/golden/*.npz: input/output vectors of the reference's own CPU
path, produced by the reference engine compiled in place from the reference
checkout (oracle/_ref/libtenzo_ref.so, built by ``make -C oracle ref``).

Run in the development container (the reference checkout is not present on
the GPU box):  python tests/golden/make_golden.py

Each fixture stores every input it was made from, so the tests never need to
regenerate inputs. Seeds are fixed per fixture.
"""
from __future__ import annotations

import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from tenzo_amd import formats, synth  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
P = oracle._ptr


def save(name, **arrays):
    path = os.path.join(OUT, name + ".npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({os.path.getsize(path)} B)")


def tl1_fixture():
    R = oracle.ref()
    rng = np.random.default_rng(101)
    out = {}
    for tag, (N, K) in {"a": (128, 2560), "b": (64, 6912), "c": (192, 64)}.items():
        tern = rng.integers(-1, 2, size=(N, K)).astype(np.int8)
        w = formats.tl1_pack(tern)
        x = rng.standard_normal(K).astype(np.float32)
        if tag == "c":
            x[5] = 0.0
            x *= np.float32(1e-7)  # below the 1e-6 absmax floor
        w_scale = synth.latent_scale(rng)
        y = np.empty(N, np.float32)
        R.ref_tl1_gemv(P(x), P(w), K, N, w_scale, P(y))
        acc = np.empty(N, np.int32)
        inv = R.ref_tl1_gemv_acc(P(x), P(w), K, N, P(acc))
        lut = np.empty(K // 2 * 32, np.int8)
        inv2 = R.ref_build_lut(P(x), K, P(lut))
        assert inv == inv2
        out.update({f"{tag}_tern": tern, f"{tag}_w": w, f"{tag}_x": x,
                    f"{tag}_w_scale": np.float32(w_scale), f"{tag}_y": y, f"{tag}_acc": acc,
                    f"{tag}_inv": np.float32(inv), f"{tag}_lut": lut})
    save("tl1_gemv", **out)


def pack_raw_fixture():
    R = oracle.ref()
    rng = np.random.default_rng(102)
    N, K = 128, 96
    tern = rng.integers(-1, 2, size=(N, K)).astype(np.int8)
    raw = formats.hf_pack_2bit(tern)
    out = np.empty(N * K // 4, np.int8)
    R.ref_pack_raw(P(raw), N, K, P(out))
    save("tl1_pack_raw", tern=tern, raw=raw, N=np.int64(N), K=np.int64(K), packed=out.view(np.uint8))


RMS_DIMS = (2560, 6912, 64, 1, 7, 13, 100, 4100)


def rmsnorm_fixture():
    """rms_norm_raw as the reference build computes it, with and without weights;
    inputs over several magnitudes (the RSQRTSS estimate's input spans binades)."""
    R = oracle.ref()
    rng = np.random.default_rng(103)
    out = {}
    for dim in RMS_DIMS:
        x = (rng.standard_normal(dim) * 3).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
        y = np.empty(dim, np.float32)
        R.ref_rms_norm(P(x), P(w), P(y), dim, np.float32(1e-5))
        y0 = np.empty(dim, np.float32)
        R.ref_rms_norm(P(x), None, P(y0), dim, np.float32(1e-5))
        out.update({f"x{dim}": x, f"w{dim}": w, f"y{dim}": y, f"ynow{dim}": y0})
    save("rmsnorm", **out)


def attention_fixture():
    R = oracle.ref()
    rng = np.random.default_rng(104)
    out = {}
    for tag, (Hq, Hkv, max_seq, pos) in {"a": (20, 5, 48, 37), "b": (4, 1, 8, 0),
                                         "c": (8, 2, 300, 299)}.items():
        D = 128
        kc = np.zeros((Hkv, max_seq, D), np.int8)
        vc = np.zeros_like(kc)
        ks = np.zeros((Hkv, max_seq), np.float32)
        vs = np.zeros_like(ks)
        if pos:
            c, s = synth.kv_quantize(rng.standard_normal((Hkv, pos, D)).astype(np.float32))
            kc[:, :pos], ks[:, :pos] = c, synth.f16_round(s)
            c, s = synth.kv_quantize(rng.standard_normal((Hkv, pos, D)).astype(np.float32))
            vc[:, :pos], vs[:, :pos] = c, synth.f16_round(s)
        q = rng.standard_normal(Hq * D).astype(np.float32)
        k = rng.standard_normal(Hkv * D).astype(np.float32)
        v = rng.standard_normal(Hkv * D).astype(np.float32)
        ins = dict(q=q.copy(), k=k.copy(), v=v.copy(), kc=kc.copy(), vc=vc.copy(),
                   ks=ks.copy(), vs=vs.copy())
        o = np.empty(Hq * D, np.float32)
        R.ref_attention_int8(Hq, Hkv, max_seq, pos, P(q), P(k), P(v), P(kc), P(vc), P(ks),
                             P(vs), P(o))
        for n, a in ins.items():
            out[f"{tag}_in_{n}"] = a
        out.update({f"{tag}_dims": np.array([Hq, Hkv, max_seq, pos], np.int64),
                    f"{tag}_out": o, f"{tag}_q_rot": q, f"{tag}_k_rot": k, f"{tag}_kc": kc,
                    f"{tag}_vc": vc, f"{tag}_ks": ks, f"{tag}_vs": vs})
    save("attention", **out)


def quant_gemv_fixture():
    R = oracle.ref()
    rng = np.random.default_rng(105)
    K, N, G = 512, 64, 128
    out = {"dims": np.array([K, N, G], np.int64)}
    a = rng.standard_normal(K).astype(np.float16).astype(np.float32)
    out["a"] = a
    # Q4_0 / Q8_0
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    d = np.abs(rng.normal(0, 0.01, size=(N, K // 32))).astype(np.float16)
    w4 = formats.q4_0_pack(q, d)
    y = np.empty(N, np.float32)
    R.ref_q4_0(P(a), P(w4), P(y), K, N)
    out.update(q4_w=w4, q4_y=y.copy())
    q8 = rng.integers(-127, 128, size=(N, K)).astype(np.int8)
    w8 = formats.q8_0_pack(q8, d)
    R.ref_q8_0(P(a), P(w8), P(y), K, N)
    out.update(q8_w=w8, q8_y=y.copy())
    # GPTQ / AWQ
    qk = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    zeros = rng.integers(0, 16, size=(K // G, N), dtype=np.uint8)
    scales = synth.f16_round(np.abs(rng.normal(0, 0.01, size=(K // G, N))))
    qw, qz = formats.gptq_pack(qk, zeros)
    R.ref_gptq(P(a), P(qw), P(scales), P(qz), P(y), K, N, G)
    out.update(gptq_qweight=qw, gptq_qzeros=qz, scales=scales, gptq_y=y.copy())
    qw, qz = formats.awq_pack(qk, zeros)
    R.ref_awq(P(a), P(qw), P(scales), P(qz), P(y), K, N, G)
    out.update(awq_qweight=qw, awq_qzeros=qz, awq_y=y.copy())
    save("quant_gemv", **out)


def layer_struct(sm, l):
    return oracle.ref_layer_struct(sm, l)


def run_ref_engine(sm, tokens):
    """Greedy steps of the compiled reference engine at theta 10000 (hard-coded there)."""
    R = oracle.ref()
    c = sm.cfg
    e = R.ref_engine_create(c.hidden, c.n_q_heads, c.n_kv_heads, c.n_layers, c.ffn, c.vocab,
                            c.max_seq)
    keep = [layer_struct(sm, l) for l in range(c.n_layers)]
    for l, w in enumerate(keep):
        assert R.ref_engine_set_layer(e, l, ctypes.byref(w)) == 0
    assert R.ref_engine_set_head(e, P(sm.embed), P(sm.embed_scales), P(sm.final_norm), c.vocab,
                                 c.hidden) == 0
    R.ref_engine_set_kv(e, P(sm.kc), P(sm.vc), P(sm.ks), P(sm.vs), sm.ctx)
    logits, hidden, out_tok = [], [], []
    for t in tokens:
        lg = np.empty(c.vocab, np.float32)
        tok = R.ref_engine_step(e, int(t), P(lg))
        h = np.empty(c.hidden, np.float32)
        R.ref_engine_hidden(e, P(h))
        logits.append(lg)
        hidden.append(h)
        out_tok.append(tok)
    kc, vc = np.empty_like(sm.kc), np.empty_like(sm.vc)
    ks, vs = np.empty_like(sm.ks), np.empty_like(sm.vs)
    R.ref_engine_get_kv(e, P(kc), P(vc), P(ks), P(vs))
    R.ref_engine_destroy(e)
    return np.array(out_tok), np.stack(logits), np.stack(hidden), (kc, vc, ks, vs)


TINY = synth.DecodeConfig(hidden=256, n_q_heads=2, n_kv_heads=1, n_layers=2, ffn=512,
                          vocab=512, max_seq=16, theta=10000.0)


def decode_fixture():
    sm = synth.make_model(TINY, seed=106, ctx=5)
    tokens = np.array([7, 300, 42], np.int64)
    out_tok, logits, hidden, (kc, vc, ks, vs) = run_ref_engine(sm, tokens)
    arrays = {"tokens": tokens, "out_tokens": out_tok, "logits": logits, "hidden": hidden,
              "kc_out": kc, "vc_out": vc, "ks_out": ks, "vs_out": vs,
              "ctx": np.int64(sm.ctx), "kc": sm.kc, "vc": sm.vc, "ks": sm.ks, "vs": sm.vs,
              "final_norm": sm.final_norm, "embed": sm.embed, "embed_scales": sm.embed_scales}
    for l, lw in enumerate(sm.layers):
        for p in synth.PROJ:
            arrays[f"l{l}_{p}"] = lw.tl1[p]
            arrays[f"l{l}_{p}_scale"] = np.float32(lw.scale[p])
        for f in ["in_norm", "attn_sub_norm", "post_norm", "ffn_sub_norm"]:
            arrays[f"l{l}_{f}"] = getattr(lw, f)
    save("decode_tiny", **arrays)


TERN_ATT = dict(Hq=8, Hkv=2, max_seq=96, pos=70)


def attention_tern_fixture():
    """FusedKVCache::forward_attention_raw in the ternary modes (1 tl1_fused,
    2 popcount_fused): the compiled reference on a random cache."""
    Hq, Hkv, S, pos = TERN_ATT["Hq"], TERN_ATT["Hkv"], TERN_ATT["max_seq"], TERN_ATT["pos"]
    cfg = synth.DecodeConfig(hidden=Hq * 128, n_q_heads=Hq, n_kv_heads=Hkv, n_layers=1, ffn=64,
                             vocab=64, max_seq=S, theta=10000.0)
    R = oracle.ref()
    out = {}
    for mode in (1, 2):
        kb, vb, ks, vs = (a[0] for a in synth.tern_kv(cfg, mode, pos, seed=20 + mode))
        rng = np.random.default_rng(30 + mode)
        q = rng.standard_normal(Hq * 128).astype(np.float32)
        k = (2 * rng.standard_normal(Hkv * 128)).astype(np.float32)
        v = rng.standard_normal(Hkv * 128).astype(np.float32)
        res = np.zeros(Hq * 128, np.float32)
        rk, rv, rks, rvs = kb.copy(), vb.copy(), ks.copy(), vs.copy()
        R.ref_attention_tern(mode, Hq, Hkv, S, pos, P(q.copy()), P(k.copy()), P(v), P(rk), P(rv),
                             P(rks), P(rvs), P(res))
        out.update({f"m{mode}_{n}": a for n, a in dict(
            q=q, k=k, v=v, kb=kb, vb=vb, ks=ks, vs=vs, out=res, kb_out=rk[:, :pos + 1],
            vb_out=rv[:, :pos + 1], ks_out=rks[:, :pos + 1], vs_out=rvs[:, :pos + 1]).items()})
    save("attention_tern", **out)


def run_ref_engine_tern(sm, mode, tokens):
    """Greedy steps of the compiled reference engine with kv_mode tl1_fused (1) /
    popcount_fused (2), from an empty cache."""
    R = oracle.ref()
    c = sm.cfg
    e = R.ref_engine_create_mode(c.hidden, c.n_q_heads, c.n_kv_heads, c.n_layers, c.ffn, c.vocab,
                                 c.max_seq, mode)
    keep = [layer_struct(sm, l) for l in range(c.n_layers)]
    for l, w in enumerate(keep):
        assert R.ref_engine_set_layer(e, l, ctypes.byref(w)) == 0
    assert R.ref_engine_set_head(e, P(sm.embed), P(sm.embed_scales), P(sm.final_norm), c.vocab,
                                 c.hidden) == 0
    logits, hidden, out_tok = [], [], []
    for t in tokens:
        lg = np.empty(c.vocab, np.float32)
        tok = R.ref_engine_step(e, int(t), P(lg))
        h = np.empty(c.hidden, np.float32)
        R.ref_engine_hidden(e, P(h))
        logits.append(lg)
        hidden.append(h)
        out_tok.append(tok)
    shape = (c.n_layers, c.n_kv_heads, c.max_seq)
    kb, vb = np.empty(shape + (32,), np.uint8), np.empty(shape + (32,), np.uint8)
    ks, vs = np.empty(shape, np.float32), np.empty(shape, np.float32)
    R.ref_engine_get_kv_tern(e, mode, P(kb), P(vb), P(ks), P(vs))
    R.ref_engine_destroy(e)
    n = len(tokens)
    return (np.array(out_tok), np.stack(logits), np.stack(hidden),
            (kb[:, :, :n], vb[:, :, :n], ks[:, :, :n], vs[:, :, :n]))


def decode_tern_fixture():
    """The decode_tiny model run by the reference engine in each ternary mode."""
    z = np.load(os.path.join(OUT, "decode_tiny.npz"))
    sm = load_tiny_model(z)
    tokens = np.array([7, 300, 42, 5, 99, 11, 250, 3], np.int64)
    out = {"tokens": tokens}
    for mode in (1, 2):
        tok, logits, hidden, (kb, vb, ks, vs) = run_ref_engine_tern(sm, mode, tokens)
        out.update({f"m{mode}_out_tokens": tok, f"m{mode}_logits": logits,
                    f"m{mode}_hidden": hidden, f"m{mode}_kb": kb, f"m{mode}_vb": vb,
                    f"m{mode}_ks": ks, f"m{mode}_vs": vs})
    save("decode_tern", **out)


PAGED_ATT = dict(Hq=8, Hkv=2, n_layers=2, layer=1, max_seq=320, pos=96)


def attention_paged_fixture():
    """PagedKVCache::forward_attention_raw on a permuted block table, position
    96 (the reference allocates the block of the new token), plus a peaked-q
    case whose softmax has weights below the 1e-7 cut-off."""
    c = PAGED_ATT
    cfg = synth.DecodeConfig(hidden=c["Hq"] * 128, n_q_heads=c["Hq"], n_kv_heads=c["Hkv"],
                             n_layers=c["n_layers"], ffn=64, vocab=64, max_seq=c["max_seq"],
                             theta=10000.0)
    nb = (c["max_seq"] + 15) // 16
    rng = np.random.default_rng(40)
    perm = rng.permutation(nb).astype(np.int32)
    pk, pv, pks, pvs = synth.paged_kv(cfg, c["pos"], perm, seed=41)
    R = oracle.ref()
    out = {"perm": perm}
    for name, qscale in (("", 1.0), ("peak_", 40.0)):
        q = (qscale * rng.standard_normal(c["Hq"] * 128)).astype(np.float32)
        k = (2 * rng.standard_normal(c["Hkv"] * 128)).astype(np.float32)
        v = rng.standard_normal(c["Hkv"] * 128).astype(np.float32)
        rc = [a.copy() for a in (pk, pv, pks, pvs)]
        bt = perm.copy()
        res = np.zeros(c["Hq"] * 128, np.float32)
        n = R.ref_attention_paged(c["Hq"], c["Hkv"], c["n_layers"], c["layer"], nb, c["pos"],
                                  P(q.copy()), P(k.copy()), P(v), *(P(a) for a in rc), P(bt),
                                  c["pos"] // 16, P(res))
        out.update({name + "q": q, name + "k": k, name + "v": v, name + "out": res,
                    name + "block_table": bt[:n], name + "pk_out": rc[0], name + "pv_out": rc[1],
                    name + "pks_out": rc[2], name + "pvs_out": rc[3]})
    out.update(pk=pk, pv=pv, pks=pks, pvs=pvs)
    save("attention_paged", **out)


def decode_paged_fixture():
    """The decode_tiny model run by the reference engine with kv_mode paged_int8
    from an empty cache (its block manager allocates as the steps go)."""
    z = np.load(os.path.join(OUT, "decode_tiny.npz"))
    sm = load_tiny_model(z)
    c = sm.cfg
    tokens = np.array([7, 300, 42, 5, 99, 11, 250, 3, 17, 64, 128, 255, 1, 2, 3, 4, 5, 6],
                      np.int64)
    R = oracle.ref()
    e = R.ref_engine_create_mode(c.hidden, c.n_q_heads, c.n_kv_heads, c.n_layers, c.ffn, c.vocab,
                                 32, 3)
    keep = [layer_struct(sm, l) for l in range(c.n_layers)]
    for l, w in enumerate(keep):
        assert R.ref_engine_set_layer(e, l, ctypes.byref(w)) == 0
    assert R.ref_engine_set_head(e, P(sm.embed), P(sm.embed_scales), P(sm.final_norm), c.vocab,
                                 c.hidden) == 0
    logits, hidden, out_tok = [], [], []
    for t in tokens:
        lg = np.empty(c.vocab, np.float32)
        out_tok.append(R.ref_engine_step(e, int(t), P(lg)))
        h = np.empty(c.hidden, np.float32)
        R.ref_engine_hidden(e, P(h))
        logits.append(lg)
        hidden.append(h)
    nb = 2
    pk = np.empty((nb, c.n_layers, c.n_kv_heads, 16, 128), np.int8)
    pv = np.empty_like(pk)
    pks = np.empty((nb, c.n_layers, c.n_kv_heads, 16), np.float32)
    pvs = np.empty_like(pks)
    bt = np.zeros(nb, np.int32)
    n = R.ref_engine_get_kv_paged(e, P(pk), P(pv), P(pks), P(pvs), P(bt))
    R.ref_engine_destroy(e)
    save("decode_paged", tokens=tokens, out_tokens=np.array(out_tok), logits=np.stack(logits),
         hidden=np.stack(hidden), pk=pk, pv=pv, pks=pks, pvs=pvs, block_table=bt[:n],
         max_seq=np.int64(32))


def load_tiny_model(z) -> synth.SynthModel:
    """Rebuilds the decode fixture's model from its stored arrays."""
    layers = []
    for l in range(TINY.n_layers):
        layers.append(synth.LayerWeights(
            {p: z[f"l{l}_{p}"] for p in synth.PROJ},
            {p: np.float32(z[f"l{l}_{p}_scale"]) for p in synth.PROJ},
            z[f"l{l}_in_norm"], z[f"l{l}_attn_sub_norm"], z[f"l{l}_post_norm"],
            z[f"l{l}_ffn_sub_norm"]))
    return synth.SynthModel(TINY, layers, z["final_norm"], z["embed"], z["embed_scales"],
                            z["kc"].copy(), z["vc"].copy(), z["ks"].copy(), z["vs"].copy(),
                            int(z["ctx"]))


if __name__ == "__main__":
    oracle.build(ref=True)
    only = sys.argv[1:]
    if only:  # e.g. python tests/golden/make_golden.py rmsnorm_fixture
        for name in only:
            globals()[name]()
        sys.exit(0)
    tl1_fixture()
    pack_raw_fixture()
    rmsnorm_fixture()
    attention_fixture()
    quant_gemv_fixture()
    decode_fixture()
    attention_tern_fixture()
    decode_tern_fixture()
    attention_paged_fixture()
    decode_paged_fixture()
