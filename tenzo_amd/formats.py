"""Host-side weight formats of the decode path (numpy, load time only).

These build the byte layouts the reference consumes, so the same bytes can be
handed to the reference CPU path and to this library's C ABI:

* TL1 ternary blocks ``[N/64][K/2][32]`` - byte ``[b][k][c]`` holds the 4-bit
  index ``(w0+1) | (w1+1) << 2`` of row ``64b+c`` for columns ``(2k, 2k+1)`` in
  its low nibble and of row ``64b+32+c`` in its high nibble
  (reference ``src/bindings/PybindModule.cpp:315-355``, consumed by
  ``src/runtime/TenzoEngine.cpp:64-146``).
* The HF BitNet 2-bit layout ``[N/4][K]`` (row ``r`` in byte ``r/4`` at shift
  ``2*(r%4)``, value ``code-1``) that ``TenzoEngine.cpp:1842-1884`` repacks.
* GGUF Q4_0 / Q8_0 blocks of 32 (``TenzoEngine.cpp:1021-1114``).
* GPTQ and AWQ int32-packed nibbles with the reference's index conventions
  (``TenzoEngine.cpp:1117-1175``).

The GPU-side TL1 layout is produced on the device by
``tenzo_hip_tl1_repack`` and is not built here.
"""
from __future__ import annotations

import numpy as np

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


# ---------------------------------------------------------------- TL1 ------

def tl1_pack(tern: np.ndarray) -> np.ndarray:
    """Dense ternary ``[N][K]`` in {-1,0,1} -> TL1 bytes ``[N/64][K/2][32]``."""
    tern = np.asarray(tern, dtype=np.int8)
    N, K = tern.shape
    if N % 64 or K % 2:
        raise ValueError("TL1 needs N % 64 == 0 and K % 2 == 0")
    u = (tern.astype(np.int16) + 1).astype(np.uint8)          # [N][K] in {0,1,2}
    idx = u[:, 0::2] | (u[:, 1::2] << 2)                       # [N][K/2]
    idx = idx.reshape(N // 64, 2, 32, K // 2)                  # [b][half][c][k]
    packed = idx[:, 0] | (idx[:, 1] << 4)                      # [b][c][k]
    return np.ascontiguousarray(packed.transpose(0, 2, 1)).reshape(-1)


def tl1_unpack(w: np.ndarray, N: int, K: int) -> np.ndarray:
    """TL1 bytes -> dense ternary ``[N][K]``."""
    w = np.asarray(w, dtype=np.uint8).reshape(N // 64, K // 2, 32)
    w = w.transpose(0, 2, 1)                                   # [b][c][k]
    halves = np.stack([w & 15, w >> 4], axis=1)                # [b][2][c][k]
    idx = halves.reshape(N, K // 2)
    out = np.empty((N, K), np.int8)
    out[:, 0::2] = (idx & 3).astype(np.int8) - 1
    out[:, 1::2] = (idx >> 2).astype(np.int8) - 1
    return out


def hf_pack_2bit(tern: np.ndarray) -> np.ndarray:
    """Dense ternary ``[N][K]`` -> the HF 2-bit layout ``[N/4][K]``."""
    tern = np.asarray(tern, dtype=np.int8)
    N, K = tern.shape
    u = (tern.astype(np.int16) + 1).astype(np.uint8).reshape(N // 4, 4, K)
    return (u[:, 0] | (u[:, 1] << 2) | (u[:, 2] << 4) | (u[:, 3] << 6)).astype(np.uint8)


def tl1_random(N: int, K: int, rng: np.random.Generator) -> np.ndarray:
    """TL1 bytes of an iid ternary matrix with P(-1)=P(0)=P(+1)=1/3."""
    v = rng.integers(0, 9, size=(2, N * K // 4), dtype=np.uint8)
    nib = (v % 3) | ((v // 3) << 2)
    return (nib[0] | (nib[1] << 4)).astype(np.uint8)


# ---------------------------------------------------------------- GGUF -----

def q4_0_pack(q: np.ndarray, d: np.ndarray) -> np.ndarray:
    """codes ``[N][K]`` in [0,15] and fp16 scales ``[N][K/32]`` -> ``[N][K/32][18]``.

    Element j < 16 of a block is the low nibble of byte j, element j >= 16
    the high nibble of byte j-16 (``TenzoEngine.cpp:1044-1057``).
    """
    q = np.asarray(q, dtype=np.uint8)
    N, K = q.shape
    qb = q.reshape(N, K // 32, 32)
    qs = qb[:, :, :16] | (qb[:, :, 16:] << 4)
    out = np.empty((N, K // 32, 18), np.uint8)
    out[:, :, :2] = np.asarray(d, dtype=np.float16).reshape(N, K // 32, 1).view(np.uint8)
    out[:, :, 2:] = qs
    return out.reshape(-1)


def q8_0_pack(q: np.ndarray, d: np.ndarray) -> np.ndarray:
    """int8 codes ``[N][K]`` and fp16 scales ``[N][K/32]`` -> ``[N][K/32][34]``."""
    q = np.asarray(q, dtype=np.int8)
    N, K = q.shape
    out = np.empty((N, K // 32, 34), np.uint8)
    out[:, :, :2] = np.asarray(d, dtype=np.float16).reshape(N, K // 32, 1).view(np.uint8)
    out[:, :, 2:] = q.reshape(N, K // 32, 32).view(np.uint8)
    return out.reshape(-1)


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """fp32 ``[K]`` -> Q8_0 blocks (llama.cpp quantize_row_q8_0: d = amax/127)."""
    x = np.asarray(x, dtype=np.float32).reshape(-1, 32)
    amax = np.abs(x).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    q = np.round(x * idv[:, None])  # numpy rounds half to even; fix ties below
    prod = (x * idv[:, None]).astype(np.float32)
    frac = np.abs(prod - np.trunc(prod))
    q = np.where(frac == 0.5, np.trunc(prod) + np.sign(prod), q)
    return q8_0_pack(q.astype(np.int8).reshape(1, -1), d.astype(np.float16).reshape(1, -1))


# ---------------------------------------------------------------- GPTQ/AWQ -

def gptq_pack(q: np.ndarray, zeros: np.ndarray):
    """Reference GPTQ layout (``TenzoEngine.cpp:1117-1143``).

    q: ``[K][N]`` codes in [0,15]; zeros: ``[G][N]`` stored zero nibbles in
    [0,15] (the kernel uses ``nibble + 1``). Returns ``qweight [K/8][N]`` u32
    (nibble e of word (k/8, n) is element k+e) and ``qzeros [G/8][N]`` u32
    (nibble g%8 of word (g/8, n) is group g).
    """
    q = np.asarray(q, dtype=np.uint32)
    K, N = q.shape
    qw = np.zeros((K // 8, N), np.uint32)
    for e in range(8):
        qw |= q[e::8] << np.uint32(4 * e)
    zeros = np.asarray(zeros, dtype=np.uint32)
    G = zeros.shape[0]
    Gp = (G + 7) // 8 * 8
    zp = np.zeros((Gp, N), np.uint32)
    zp[:G] = zeros
    qz = np.zeros((Gp // 8, N), np.uint32)
    for e in range(8):
        qz |= zp[e::8] << np.uint32(4 * e)
    return qw, qz


def awq_pack(q: np.ndarray, zeros: np.ndarray):
    """Reference AWQ layout (``TenzoEngine.cpp:1146-1175``).

    q: ``[K][N]`` codes; zeros ``[G][N]`` in [0,15] (used as is). Nibble e of
    ``qweight[k/8][n]`` is element ``k + AWQ_ORDER[e]``; ``qzeros[g][n/8]``
    holds column n's zero in nibble n%8.
    """
    q = np.asarray(q, dtype=np.uint32)
    K, N = q.shape
    qw = np.zeros((K // 8, N), np.uint32)
    for e, o in enumerate(AWQ_ORDER):
        qw |= q[o::8] << np.uint32(4 * e)
    zeros = np.asarray(zeros, dtype=np.uint32)
    G = zeros.shape[0]
    qz = np.zeros((G, N // 8), np.uint32)
    for e in range(8):
        qz |= zeros[:, e::8] << np.uint32(4 * e)
    return qw, qz
