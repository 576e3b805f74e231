"""Writes a weights.bin + model.mlir pair in the layout the reference's
tenzo_load_model reads (load_model_from_files, TenzoEngine.cpp:1887-2078) and
its BitNet exporter writes (tenzo-frontend/export_output/model.mlir): the fp32
embedding table at offset 0, then per layer in_norm, q, k, v, attn_sub_norm,
out, post_norm, gate, up, ffn_sub_norm, down, then the final norm. Ternary
projections are raw [N/4][K] bytes (row r of column c at bits 2(r%4) as w+1);
each tensor is announced by an index constant + memref.view pair and each
projection's scale by an f32 constant + "tenzo.bitlinear_elut" pair. Test
infrastructure."""
from __future__ import annotations

import os

import numpy as np

ORDER = ["in_norm", "q", "k", "v", "attn_sub_norm", "out", "post_norm", "gate", "up",
         "ffn_sub_norm", "down"]


def raw_ternary(N, K, rng):
    """Random ternary [N][K] and its raw [N/4][K] bytes."""
    t = rng.integers(-1, 2, (N, K)).astype(np.int8)
    u = (t + 1).astype(np.uint8).reshape(N // 4, 4, K)
    raw = u[:, 0] | (u[:, 1] << 2) | (u[:, 2] << 4) | (u[:, 3] << 6)
    return t, np.ascontiguousarray(raw, np.uint8)


def write(dirpath, H=2560, Hq=20, Hkv=5, F=512, L=2, V=320, seed=0, views="all",
          truncate=None):
    """Returns (weights_path, mlir_path, tensors) with tensors[l][name] the
    arrays written and tensors['embed'], tensors['final_norm'].
    views: "all" announces every tensor; an int k announces only the first k
    views (the loader then continues at sequential offsets). truncate: cut
    weights.bin to that many bytes."""
    rng = np.random.default_rng(seed)
    qd, kvd = Hq * 128, Hkv * 128
    shapes = {"q": (qd, H), "k": (kvd, H), "v": (kvd, H), "out": (H, qd), "gate": (F, H),
              "up": (F, H), "down": (H, F)}
    blobs, tensors = [], {}
    embed = (rng.standard_normal((V, H)) * 0.02).astype(np.float32)
    tensors["embed"] = embed
    blobs.append(("embed", embed.tobytes(), f"{V}x{H}xf32", None))
    for l in range(L):
        tl = {}
        for name in ORDER:
            if name.endswith("norm"):
                n = F if name == "ffn_sub_norm" else H
                v = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
                tl[name] = v
                blobs.append((f"{l}.{name}", v.tobytes(), f"{n}xf32", None))
            else:
                N, K = shapes[name]
                t, raw = raw_ternary(N, K, rng)
                scale = np.float32(rng.uniform(0.5, 3.0))
                tl[name] = (t, raw, scale)
                blobs.append((f"{l}.{name}", raw.tobytes(), f"{N}x{K // 4}xi8", scale))
        tensors[l] = tl
    fin = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    tensors["final_norm"] = fin
    blobs.append(("final_norm", fin.tobytes(), f"{H}xf32", None))

    wpath = os.path.join(dirpath, "weights.bin")
    mpath = os.path.join(dirpath, "model.mlir")
    lines = ["// synthetic model in the Tenzo BitNet exporter's layout", "module {",
             "  func.func @main(%arg0: tensor<1x1xi32>, %arg1: memref<?xi8>) {"]
    off, k = 0, 0
    nviews = len(blobs) if views == "all" else int(views)
    with open(wpath, "wb") as f:
        for i, (name, data, shape, scale) in enumerate(blobs):
            f.write(data)
            if i < nviews:
                lines.append(f"    %v{k} = arith.constant {off} : index")
                lines.append(f"    %v{k + 1} = memref.view %arg1[%v{k}][] : memref<?xi8> to "
                             f"memref<{shape}>")
                lines.append(f"    %v{k + 2} = bufferization.to_tensor %v{k + 1} : "
                             f"memref<{shape}>")
                k += 3
            if scale is not None:
                lines.append(f"    %v{k} = arith.constant {float(scale):.8e} : f32")
                lines.append(f'    %v{k + 1} = "tenzo.bitlinear_elut"(%x, %v{k - 1}, %v{k}) '
                             '{bit_width = 2 : i32, quant_scheme = "ternary"} : '
                             "(tensor<1x1xf32>, tensor<1xi8>, f32) -> tensor<1x1xf32>")
                k += 2
            off += len(data)
    lines += ["    return", "  }", "}"]
    with open(mpath, "w") as f:
        f.write("\n".join(lines) + "\n")
    if truncate is not None:
        with open(wpath, "r+b") as f:
            f.truncate(truncate)
    return wpath, mpath, tensors
