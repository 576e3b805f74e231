"""The drop-in boundary as a C++ caller sees it: a program written against
include/ only (tenzo.hpp over tenzo.h, the reference SDK's interface) is built
with g++, linked against libtenzo_hip.so, loads a model from weights.bin +
model.mlir, prefills a prompt and decodes greedily; its tokens equal the CPU
oracle's on the same model."""
import os
import subprocess

import numpy as np
import pytest

import oracle
from tenzo_amd import synth
from tests import model_files

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def oracle_model(t, cfg):
    layers = []
    for l in range(cfg.n_layers):
        tl = t[l]
        tl1 = {p: oracle.tl1_pack(tl[n][0]) for p, n in
               (("q", "q"), ("k", "k"), ("v", "v"), ("o", "out"), ("gate", "gate"), ("up", "up"),
                ("down", "down"))}
        scale = {p: np.float32(tl[n][2]) for p, n in
                 (("q", "q"), ("k", "k"), ("v", "v"), ("o", "out"), ("gate", "gate"),
                  ("up", "up"), ("down", "down"))}
        layers.append(synth.LayerWeights(tl1, scale, tl["in_norm"], tl["attn_sub_norm"],
                                         tl["post_norm"], tl["ffn_sub_norm"]))
    embed, es = oracle.quant_rows_i8(t["embed"])
    shape = (cfg.n_layers, cfg.n_kv_heads, cfg.max_seq, 128)
    z8, z32 = np.zeros(shape, np.int8), np.zeros(shape[:3], np.float32)
    return synth.SynthModel(cfg, layers, t["final_norm"], embed, es, z8, z8.copy(), z32,
                            z32.copy(), 0)


def test_cxx_caller_through_tenzo_hpp(tmp_path):
    import torch
    assert torch.cuda.is_available(), "GPU test needs a visible GPU"
    H, Hq, Hkv, L, F, V, S = 512, 4, 1, 2, 512, 300, 32
    wpath, mpath, t = model_files.write(str(tmp_path), H=H, Hq=Hq, Hkv=Hkv, F=F, L=L, V=V, seed=9)
    exe = str(tmp_path / "tenzo_caller")
    cmd = ["g++", "-std=c++17", "-O2", "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "cxx", "tenzo_caller.cpp"),
           "-L", os.path.join(ROOT, "tenzo_amd"), "-ltenzo_hip",
           "-Wl,-rpath," + os.path.join(ROOT, "tenzo_amd"), "-Wl,-rpath,/opt/rocm/lib",
           "-L/opt/rocm/lib", "-o", exe]
    print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True, timeout=120)
    prompt, n_gen = [7, 200, 13, 64, 5], 6
    r = subprocess.run([exe, wpath, mpath, str(H), str(Hq), str(Hkv), str(L), str(F), str(V),
                        str(S), str(n_gen)] + [str(p) for p in prompt],
                       capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0
    got = [int(v) for v in r.stdout.split()]
    cfg = synth.DecodeConfig(hidden=H, n_q_heads=Hq, n_kv_heads=Hkv, n_layers=L, ffn=F, vocab=V,
                             max_seq=S, theta=10000.0)
    om = oracle.OracleModel(oracle_model(t, cfg), f16_kv_scales=True)
    for i, p in enumerate(prompt[:-1]):
        om.step(p, i, cfg.theta)
    tok, ref = prompt[-1], []
    for i in range(n_gen):
        tok = om.step(tok, len(prompt) - 1 + i, cfg.theta)[0]
        ref.append(tok)
    assert got == ref
    assert f"seq_len {len(prompt) - 1 + n_gen}" in r.stderr
