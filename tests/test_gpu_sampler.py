"""The device sampler (sample_top_k_top_p, TenzoEngine.cpp:1722-1807, temperature
> 0) against the oracle restatement, which is itself pinned against the
compiled reference's sampler on the same rand() draws (tests/test_oracle.py).
Tokens must be equal; the only freedom is the last ulp of expf, which can move
a draw that sits on a cumulative-probability boundary (none in these cases)."""
import ctypes

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU test needs a visible GPU"
    from tenzo_amd import _lib
    _lib.load()
    return torch


def _libc():
    libc = ctypes.CDLL("libc.so.6")
    libc.rand.restype = ctypes.c_int
    libc.srand.argtypes = [ctypes.c_uint]
    return libc


@pytest.mark.parametrize("V", [17, 1000, 2048, 2049, 50000, 128256, 262144])
def test_sampler_matches_oracle(torch_dev, V):
    from tenzo_amd import ops
    torch = torch_dev
    rng = np.random.default_rng(V)
    cases = [(40, 0.9, 0.7), (1, 0.9, 0.7), (64, 1.0, 1.3), (10, 0.5, 0.2), (64, 0.99, 5.0),
             (3, 0.1, 1.0), (200, 0.95, 0.8), (0, 0.9, 0.7)]
    print(f"sampler V={V}", flush=True)
    for trial in range(24):
        k, p, T = cases[trial % len(cases)]
        logits = (rng.standard_normal(V) * rng.uniform(0.5, 8.0)).astype(np.float32)
        r = float(np.float32(rng.uniform(0, 1)))
        got = ops.sample_top_k_top_p(torch.from_numpy(logits).cuda(), k, p, T, r)
        want = oracle.sample_top_k_top_p(logits, k, p, T, r)
        assert got == want, (trial, k, p, T, r)


def test_sampler_edge_draws(torch_dev):
    """r = 0 picks the largest logit, r = 1 the last candidate inside the
    top-p cutoff; -inf logits are never drawn; V smaller than k."""
    from tenzo_amd import ops
    torch = torch_dev
    rng = np.random.default_rng(1)
    logits = rng.standard_normal(5000).astype(np.float32)
    d = torch.from_numpy(logits).cuda()
    for k, p, T in [(40, 0.9, 0.7), (64, 1.0, 2.0), (5, 0.3, 0.5)]:
        for r in (0.0, 1.0, 0.5):
            assert ops.sample_top_k_top_p(d, k, p, T, r) == oracle.sample_top_k_top_p(
                logits, k, p, T, r)
    masked = np.full(3000, -np.inf, np.float32)
    masked[[7, 1999, 2500]] = [1.0, 3.0, 2.0]
    for r in (0.0, 0.3, 0.9, 1.0):
        t = ops.sample_top_k_top_p(torch.from_numpy(masked).cuda(), 64, 1.0, 1.0, r)
        assert t in (7, 1999, 2500)
        assert t == oracle.sample_top_k_top_p(masked, 64, 1.0, 1.0, r)
    small = np.array([0.5, 2.0, -1.0], np.float32)
    assert ops.sample_top_k_top_p(torch.from_numpy(small).cuda(), 40, 0.9, 1.0, 0.99) == \
        oracle.sample_top_k_top_p(small, 40, 0.9, 1.0, 0.99)


@pytest.mark.parametrize("mode", ["persistent", "eager"])
def test_engine_generate_step_samples(torch_dev, mode):
    """tenzo_generate_step with temperature > 0: the engine draws r from the
    process's rand() like the reference; reseeding libc and replaying the
    oracle sampler on the engine's (penalised) logits gives the same token."""
    from tenzo_amd import engine as eng_mod, synth
    libc = _libc()
    cfg = synth.DecodeConfig(hidden=512, n_q_heads=4, n_kv_heads=1, n_layers=2, ffn=512,
                             vocab=4096, max_seq=64, theta=10000.0)
    sm = synth.make_model(cfg, seed=19, ctx=6)
    with eng_mod.Engine(cfg) as e:
        e.set_model(sm)
        e.set_mode(mode)
        past = [3, 9, 27, 3]
        tok = 5
        for i, (T, k, p, pen) in enumerate([(0.8, 40, 0.9, 1.15), (1.5, 64, 0.99, 1.0),
                                            (0.3, 8, 0.5, 1.3), (2.0, 1, 0.9, 1.0)]):
            libc.srand(77 + i)
            got = e.step(tok, temperature=T, penalty=pen, past=past, top_k=k, top_p=p)
            logits = e.logits()  # the penalised logits the sampler saw
            libc.srand(77 + i)
            r = np.float32(libc.rand()) / np.float32(2147483647)
            assert got == oracle.sample_top_k_top_p(logits, k, p, T, float(r)), (i, mode)
            past.append(got)
            tok = got
