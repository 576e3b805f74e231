"""The paged_int8 KV mode of the oracle (PagedKVCache, TenzoEngine.cpp:218-445)
pinned against the compiled reference (its fixture and, where built, live) and
the paging invariance (the same tokens through any block table give the same
result). Bars: pool rows and scales bit-exact, outputs 1e-5."""
import os

import numpy as np
import pytest

import oracle
from tenzo_amd import synth

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
HQ, HKV, NL, LAYER, S, POS = 8, 2, 2, 1, 320, 96  # make_golden.PAGED_ATT


def rel(a, b):
    return np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30)


@pytest.mark.parametrize("case", ["", "peak_"])
def test_oracle_matches_reference_fixture(case):
    """"peak_": a q scaled 40x, so most softmax weights fall below the 1e-7
    cut-off (the reference skips their values)."""
    z = np.load(os.path.join(GOLD, "attention_paged.npz"))
    pools = [z[n].copy() for n in ("pk", "pv", "pks", "pvs")]
    out, _, _ = oracle.attention_step_paged(z[case + "q"], z[case + "k"], z[case + "v"], *pools,
                                            z[case + "block_table"], NL, LAYER, HQ, HKV, POS,
                                            oracle.rope_table(10000.0, POS))
    for a, n in zip(pools, ("pk", "pv", "pks", "pvs")):
        np.testing.assert_array_equal(a, z[case + n + "_out"])
    assert rel(out, z[case + "out"]) < 1e-5
    if case:
        p = z[case + "q"]  # the cut-off is exercised: many weights are tiny
        assert np.abs(p).max() > 50


@pytest.mark.skipif(not oracle.ref_available(), reason="compiled reference not built")
@pytest.mark.parametrize("Hq,Hkv,L,layer,S,pos", [(4, 1, 1, 0, 64, 0), (20, 5, 2, 1, 640, 600),
                                                  (16, 2, 1, 0, 2048, 2000), (8, 8, 1, 0, 256, 47),
                                                  (8, 2, 2, 1, 320, 64)])
def test_oracle_matches_compiled_reference(Hq, Hkv, L, layer, S, pos):
    P = oracle._ptr
    cfg = synth.DecodeConfig(hidden=Hq * 128, n_q_heads=Hq, n_kv_heads=Hkv, n_layers=L, ffn=64,
                             vocab=64, max_seq=S, theta=10000.0)
    nb = (S + 15) // 16
    rng = np.random.default_rng(pos)
    perm = rng.permutation(nb).astype(np.int32)
    pk, pv, pks, pvs = synth.paged_kv(cfg, pos, perm, seed=pos)
    q = rng.standard_normal(Hq * 128).astype(np.float32)
    k = (2 * rng.standard_normal(Hkv * 128)).astype(np.float32)
    v = rng.standard_normal(Hkv * 128).astype(np.float32)
    rc = [a.copy() for a in (pk, pv, pks, pvs)]
    bt = perm.copy()
    ro = np.zeros(Hq * 128, np.float32)
    n = oracle.ref().ref_attention_paged(Hq, Hkv, L, layer, nb, pos, P(q.copy()), P(k.copy()),
                                         P(v), *(P(a) for a in rc), P(bt), (pos + 15) // 16, P(ro))
    oc = [a.copy() for a in (pk, pv, pks, pvs)]
    out, _, _ = oracle.attention_step_paged(q, k, v, *oc, bt[:n], L, layer, Hq, Hkv, pos,
                                            oracle.rope_table(10000.0, pos))
    for a, b in zip(oc, rc):
        np.testing.assert_array_equal(a, b)
    assert rel(out, ro) < 1e-5


def test_paging_invariance():
    """The same tokens placed through an identity and a permuted block table
    give bit-identical outputs and the same logical rows."""
    cfg = synth.DecodeConfig(hidden=1024, n_q_heads=8, n_kv_heads=2, n_layers=2, ffn=64,
                             vocab=64, max_seq=256, theta=10000.0)
    pos = 150
    ident = np.arange(16, dtype=np.int32)
    perm = np.random.default_rng(3).permutation(16).astype(np.int32)
    outs, rows = [], []
    for bt in (ident, perm):
        pools = list(synth.paged_kv(cfg, pos, bt, seed=9))
        rng = np.random.default_rng(1)
        q = rng.standard_normal(1024).astype(np.float32)
        k = rng.standard_normal(256).astype(np.float32)
        v = rng.standard_normal(256).astype(np.float32)
        out, _, _ = oracle.attention_step_paged(q, k, v, *pools, bt, 2, 1, 8, 2, pos,
                                                oracle.rope_table(10000.0, pos))
        outs.append(out)
        rows.append(pools[0][bt[pos // 16], 1, :, pos % 16].copy())
    np.testing.assert_array_equal(outs[0], outs[1])
    np.testing.assert_array_equal(rows[0], rows[1])
