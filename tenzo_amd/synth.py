"""Seeded synthetic inputs for the decode path (the shapes of the five
benchmark configurations; no checkpoints or datasets are used).

Small configurations are generated with numpy on the host (tests, smoke);
full-size tensors for the benchmark are generated on the device with torch
(see ``bench.py``), following the same recipes:

* TL1 weights: iid ternary, P(-1)=P(0)=P(+1)=1/3, packed to TL1 blocks; the
  per-tensor scale is mean|Z| of an N(0, 0.02) latent, estimated on a 65,536
  sample per tensor.
* LM head / tied embedding: latent E ~ N(0, 0.02); per-row scale
  ``max(1e-8, max|E_v|)/127``; codes ``clamp(round(E/s), -127, 127)`` - the
  quantization ``load_model_from_files`` applies (reference
  ``TenzoEngine.cpp:1929-1946``).
* INT8 KV cache: K, V ~ N(0, 1) per (layer, kv-head, token), quantized with
  the cache's own rule (``TenzoEngine.cpp:516-531``), scales kept as fp16.
* RMSNorm weights: 1 + 0.1 N(0, 1) (the reference ships trained norms; any
  positive vector exercises the same arithmetic).
"""
from __future__ import annotations

import dataclasses

import numpy as np

from . import formats

HEAD_DIM = 128
PROJ = ("q", "k", "v", "o", "gate", "up", "down")


@dataclasses.dataclass(frozen=True)
class DecodeConfig:
    hidden: int = 2560
    n_q_heads: int = 20
    n_kv_heads: int = 5
    n_layers: int = 30
    ffn: int = 6912
    vocab: int = 128256
    max_seq: int = 8192
    eps: float = 1e-5
    theta: float = 500000.0

    @property
    def q_dim(self) -> int:
        return self.n_q_heads * HEAD_DIM

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * HEAD_DIM

    def proj_shape(self, name: str):
        """(N, K) of a projection."""
        H, F = self.hidden, self.ffn
        return {
            "q": (self.q_dim, H), "k": (self.kv_dim, H), "v": (self.kv_dim, H),
            "o": (H, self.q_dim), "gate": (F, H), "up": (F, H), "down": (H, F),
        }[name]

    def step_bytes(self, ctx: int, kv_scale_bytes: int = 2) -> dict:
        """Algorithmic HBM bytes of one decode step at context ``ctx``."""
        tl1 = sum(n * k // 4 for n, k in (self.proj_shape(p) for p in PROJ)) * self.n_layers
        head = self.vocab * self.hidden + self.vocab * 4
        kv = self.n_layers * self.n_kv_heads * ctx * (2 * HEAD_DIM + 2 * kv_scale_bytes)
        norms = (self.n_layers * (3 * self.hidden + self.ffn) + self.hidden) * 4
        embed = self.hidden
        return {"tl1": tl1, "lm_head": head, "kv": kv, "norms": norms, "embed": embed,
                "total": tl1 + head + kv + norms + embed}


BITNET_2B = DecodeConfig()
# A small configuration with the same structure (GQA 4:1, head_dim 128).
SMALL = DecodeConfig(hidden=512, n_q_heads=4, n_kv_heads=1, n_layers=2, ffn=1024, vocab=2048,
                     max_seq=64, theta=10000.0)


def f16_round(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def latent_scale(rng: np.random.Generator, sample: int = 65536) -> np.float32:
    z = rng.normal(0.0, 0.02, size=sample).astype(np.float32)
    return np.float32(np.abs(z).mean())


def kv_quantize(x: np.ndarray):
    """Per-row (last axis) KV quantization: fp32 scale and codes (numpy).

    Same rule as the cache append as the reference build evaluates it:
    ``s = max(1e-8, amax) * (1/127)``, ``codes = clamp(round(x * (127/amax)),
    -128, 127)``, round half away from zero.
    """
    x = np.asarray(x, np.float32)
    amax = np.maximum(np.float32(1e-8), np.abs(x).max(axis=-1)).astype(np.float32)
    s = (amax * np.float32(1.0 / 127.0)).astype(np.float32)
    inv = (np.float32(127.0) / amax).astype(np.float32)
    p = (x * inv[..., None]).astype(np.float32)
    r = np.where(np.abs(p - np.trunc(p)) == 0.5, np.trunc(p) + np.sign(p), np.round(p))
    return np.clip(r, -128, 127).astype(np.int8), s


def head_quantize(E: np.ndarray):
    """LM-head quantization of ``load_model_from_files`` (clamp to +-127)."""
    E = np.asarray(E, np.float32)
    amax = np.maximum(np.float32(1e-8), np.abs(E).max(axis=1)).astype(np.float32)
    s = (amax * np.float32(1.0 / 127.0)).astype(np.float32)
    inv = (np.float32(127.0) / amax).astype(np.float32)
    p = (E * inv[:, None]).astype(np.float32)
    r = np.where(np.abs(p - np.trunc(p)) == 0.5, np.trunc(p) + np.sign(p), np.round(p))
    return np.clip(r, -127, 127).astype(np.int8), s


@dataclasses.dataclass
class LayerWeights:
    tl1: dict
    scale: dict
    in_norm: np.ndarray
    attn_sub_norm: np.ndarray
    post_norm: np.ndarray
    ffn_sub_norm: np.ndarray


@dataclasses.dataclass
class SynthModel:
    cfg: DecodeConfig
    layers: list
    final_norm: np.ndarray
    embed: np.ndarray          # [vocab][hidden] int8 (tied LM head)
    embed_scales: np.ndarray   # [vocab] fp32
    kc: np.ndarray             # [L][Hkv][max_seq][128] int8
    vc: np.ndarray
    ks: np.ndarray             # [L][Hkv][max_seq] fp32 (fp16-representable)
    vs: np.ndarray
    ctx: int                   # tokens already in the cache


def make_model(cfg: DecodeConfig, seed: int = 2, ctx: int = 0) -> SynthModel:
    """A random-init model of ``cfg`` with ``ctx`` tokens prefilled in the cache."""
    rng = np.random.default_rng(seed)
    layers = []
    for _ in range(cfg.n_layers):
        tl1, scale = {}, {}
        for p in PROJ:
            N, K = cfg.proj_shape(p)
            tl1[p] = formats.tl1_random(N, K, rng)
            scale[p] = latent_scale(rng)

        def norm(n):
            return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)

        layers.append(LayerWeights(tl1, scale, norm(cfg.hidden), norm(cfg.hidden),
                                   norm(cfg.hidden), norm(cfg.ffn)))
    final_norm = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    E = rng.normal(0.0, 0.02, size=(cfg.vocab, cfg.hidden)).astype(np.float32)
    embed, embed_scales = head_quantize(E)
    shape = (cfg.n_layers, cfg.n_kv_heads, cfg.max_seq, HEAD_DIM)
    kc = np.zeros(shape, np.int8)
    vc = np.zeros(shape, np.int8)
    ks = np.zeros(shape[:3], np.float32)
    vs = np.zeros(shape[:3], np.float32)
    if ctx:
        for arr_c, arr_s in ((kc, ks), (vc, vs)):
            x = rng.standard_normal((cfg.n_layers, cfg.n_kv_heads, ctx, HEAD_DIM)).astype(np.float32)
            c, s = kv_quantize(x)
            arr_c[:, :, :ctx] = c
            arr_s[:, :, :ctx] = f16_round(s)
    return SynthModel(cfg, layers, final_norm, embed, embed_scales, kc, vc, ks, vs, ctx)


def tern_kv(cfg: DecodeConfig, mode: int, ctx: int, seed: int = 3):
    """Random ternary KV cache content for ``ctx`` tokens (mode 1 tl1_fused,
    2 popcount_fused): rows [L][Hkv][max_seq][32] uint8 and fp32 scales
    [L][Hkv][max_seq]. Each dim is -1 / 0 / +1 with probabilities 0.345 /
    0.31 / 0.345 (a Gaussian row thresholded at half its mean |x|); scales
    around the mean |x| above that threshold."""
    rng = np.random.default_rng(seed)
    shape = (cfg.n_layers, cfg.n_kv_heads, cfg.max_seq)
    rows = {}
    for name in ("k", "v"):
        w = rng.choice(np.array([-1, 0, 1], np.int8), size=shape[:2] + (ctx, HEAD_DIM),
                       p=[0.345, 0.31, 0.345])
        if name == "k" and mode == 2:
            pos, neg = w > 0, w < 0
            planes = [np.packbits(m[..., h * 64:(h + 1) * 64], axis=-1, bitorder="little")
                      for m in (pos, neg) for h in (0, 1)]
            packed = np.concatenate(planes, axis=-1)  # kp0 | kp1 | kn0 | kn1
        else:
            f = (w + 1).astype(np.uint8).reshape(shape[:2] + (ctx, HEAD_DIM // 4, 4))
            packed = f[..., 0] | (f[..., 1] << 2) | (f[..., 2] << 4) | (f[..., 3] << 6)
        full = np.zeros(shape + (32,), np.uint8)
        full[:, :, :ctx] = packed
        sc = np.zeros(shape, np.float32)
        sc[:, :, :ctx] = rng.uniform(0.9, 1.5, size=shape[:2] + (ctx,)).astype(np.float32)
        rows[name] = (full, sc)
    return rows["k"][0], rows["v"][0], rows["k"][1], rows["v"][1]


PAGE = 16  # tokens per block of the paged_int8 cache


def paged_kv(cfg: DecodeConfig, ctx: int, block_table, seed: int = 4):
    """Random paged_int8 pools for ``ctx`` tokens placed through ``block_table``:
    codes [blocks][L][Hkv][16][128] int8 (per-token quantized N(0,1) rows) and
    fp32 scales [blocks][L][Hkv][16], blocks = ceil(max_seq / 16)."""
    rng = np.random.default_rng(seed)
    nb = (cfg.max_seq + PAGE - 1) // PAGE
    L, Hkv = cfg.n_layers, cfg.n_kv_heads
    pools = []
    for _ in range(2):
        codes = np.zeros((nb, L, Hkv, PAGE, HEAD_DIM), np.int8)
        scales = np.ones((nb, L, Hkv, PAGE), np.float32)
        if ctx:
            c, sc = kv_quantize(rng.standard_normal((L, Hkv, ctx, HEAD_DIM)).astype(np.float32))
            for t in range(ctx):
                codes[block_table[t // PAGE], :, :, t % PAGE] = c[:, :, t]
                scales[block_table[t // PAGE], :, :, t % PAGE] = sc[:, :, t]
        pools += [codes, scales]
    return pools[0], pools[2], pools[1], pools[3]
