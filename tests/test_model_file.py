"""tenzo_load_model's file reading on the CPU: the model.mlir scan against the
reference's own patterns and the reference's shipped BitNet-2B export, and the
oracle's view of a loaded model against the compiled reference's loader
(load_model_from_files, TenzoEngine.cpp:1887-2078)."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle
from tests import model_files

REF_MLIR = "/root/reference/tenzo-frontend/export_output/model.mlir"
# ref_engine_layer_data's selector: the seven projections, then the four norms
WHICH = {"q": 0, "k": 1, "v": 2, "out": 3, "gate": 4, "up": 5, "down": 6, "in_norm": 7,
         "attn_sub_norm": 8, "post_norm": 9, "ffn_sub_norm": 10}

# The two statement pairs load_model_from_files matches (TenzoEngine.cpp:1945,1953),
# as Python regular expressions: an independent reading of the same format.
VIEW_RE = re.compile(r"(%\w+)\s*=\s*arith\.constant\s+(\d+)\s*:\s*index\s*\r?\n\s*(%\w+)\s*=\s*"
                     r"memref\.view\s+%\w+\[\1\]\[\]\s*:\s*memref<\?xi8>\s+to\s+memref<([^>]+)>")
SCALE_RE = re.compile(r"(%\w+)\s*=\s*arith\.constant\s+([0-9\.e\+\-]+)\s*:\s*f32\s*\r?\n\s*%\w+"
                      r"\s*=\s*\"tenzo\.bitlinear_elut\"\([^,]+,\s*[^,]+,\s*\1\)")


def parse(text: str):
    from tenzo_amd import _lib
    L = _lib.load()
    views = np.zeros(4096, np.uint64)
    scales = np.zeros(4096, np.float32)
    nv, ns = ctypes.c_int(), ctypes.c_int()
    assert L.tenzo_hip_parse_model_mlir(text.encode(), views.ctypes.data, 4096,
                                        scales.ctypes.data, 4096, ctypes.byref(nv),
                                        ctypes.byref(ns)) == 0
    return [int(v) for v in views[:nv.value]], scales[:ns.value].copy()


def parse_re(text: str):
    return ([int(m.group(2)) for m in VIEW_RE.finditer(text)],
            np.array([np.float32(float(m.group(2))) for m in SCALE_RE.finditer(text)], np.float32))


@pytest.mark.skipif(not os.path.exists(REF_MLIR), reason="reference export not present")
def test_parse_shipped_bitnet_export():
    """The reference's own 30-layer BitNet-2B export: 332 views (embedding, 11
    per layer, final norm) at consecutive offsets whose gaps are exactly the
    tensor sizes of the loader's order, and 210 positive scales (7 per layer)."""
    text = open(REF_MLIR).read()
    views, scales = parse(text)
    rv, rs = parse_re(text)
    assert views == rv and np.array_equal(scales, rs)
    assert len(views) == 1 + 30 * 11 + 1 and len(scales) == 30 * 7
    H, F, V, qd, kvd = 2560, 6912, 128256, 2560, 640
    sizes = {"in_norm": H * 4, "q": qd * H // 4, "k": kvd * H // 4, "v": kvd * H // 4,
             "attn_sub_norm": H * 4, "out": H * qd // 4, "post_norm": H * 4,
             "gate": F * H // 4, "up": F * H // 4, "ffn_sub_norm": F * 4, "down": H * F // 4}
    expect = [0, V * H * 4]
    for _ in range(30):
        for name in model_files.ORDER:
            expect.append(expect[-1] + sizes[name])
    assert views == expect
    assert (scales > 0).all()


@pytest.mark.parametrize("text", [
    "%a = arith.constant 5 : index\n%b = memref.view %x[%a][] : memref<?xi8> to memref<4xf32>",
    "%a = arith.constant 5 : index\r\n  %b = memref.view %x[%a][] : memref<?xi8> to memref<4xf32>",
    "%a = arith.constant 5 : index\n\n\n   %b = memref.view %x[%a][] : memref<?xi8> to memref<2x2xi8>",
    "%a = arith.constant 5 : index   \n%b=memref.view  %x[%a][]:memref<?xi8>  to  memref<1xf32>",
    "%a = arith.constant 5 : index %b = memref.view %x[%a][] : memref<?xi8> to memref<4xf32>",
    "%a = arith.constant 5 : index\n%b = memref.view %x[%c][] : memref<?xi8> to memref<4xf32>",
    "%a = arith.constant 5 : index\nfoo\n%b = memref.view %x[%a][] : memref<?xi8> to memref<4xf32>",
    "%a1 = arith.constant 7 : index\n%b = memref.view %x[%a][] : memref<?xi8> to memref<4xf32>",
    "%a = arith.constant -5 : index\n%b = memref.view %x[%a][] : memref<?xi8> to memref<4xf32>",
    "%s = arith.constant 1.5e+00 : f32\n%r = \"tenzo.bitlinear_elut\"(%p, %q, %s) {x}",
    "%s = arith.constant -2.5e-01 : f32\n  %r = \"tenzo.bitlinear_elut\"(%p,%q,%s)",
    "%s = arith.constant 1.5 : f32\n%r = \"tenzo.bitlinear_elut\"(%p, %q, %s1)",
    "%s = arith.constant 1.5 : f32\n%r = \"tenzo.bitlinear_elut\"(%p, %s)",
    "%s = arith.constant 1.5 : f32 %r = \"tenzo.bitlinear_elut\"(%p, %q, %s)",
    "%s = arith.constant 1.5E+00 : f32\n%r = \"tenzo.bitlinear_elut\"(%p, %q, %s)",
    "x %a = arith.constant 3 : index\n%b = memref.view %y[%a][] : memref<?xi8> to memref<8xi8>"
    "\n%c = arith.constant 9 : index\n%d = memref.view %y[%c][] : memref<?xi8> to memref<8xi8>",
])
def test_parse_edge_cases_agree_with_the_reference_patterns(text):
    views, scales = parse(text)
    rv, rs = parse_re(text)
    assert views == rv
    assert np.array_equal(scales, rs)


@pytest.mark.skipif(not oracle.ref_available(), reason="compiled reference not built")
@pytest.mark.parametrize("variant", ["all", "views5", "truncated"])
def test_loader_matches_compiled_reference(tmp_path, variant):
    """The compiled reference loads synthetic files (seeds whose embedding
    holds exact .5 rounding ties); what it stores (TL1 blocks,
    scales, norms, the int8 LM head) equals the oracle's reading of the same
    files through this repo's MLIR scan: pack_ternary_weights_raw = the
    oracle's orc_tl1_pack_raw, the head = orc_quant_rows_i8. With 5 views only
    the loader falls back to sequential offsets; with the file cut inside
    layer 1 it falls back to zero weights (0x55 TL1 bytes) and unit norms."""
    H, Hq, Hkv, F, L, V = 2560, 20, 5, 512, 2, 320
    kw = {"views": 5} if variant == "views5" else {}
    if variant == "truncated":
        kw["truncate"] = V * H * 4 + 5_000_000
    wpath, mpath, T = model_files.write(str(tmp_path), H=H, Hq=Hq, Hkv=Hkv, F=F, L=L, V=V,
                                        seed=13, **kw)
    R = oracle.ref()
    e = R.ref_engine_create(H, Hq, Hkv, L, F, V, 16)
    try:
        assert R.ref_engine_load(e, wpath.encode(), mpath.encode()) == 0
        raw = np.fromfile(wpath, np.uint8)
        views, scales = parse(open(mpath).read())
        sizes = {"q": (Hq * 128, H), "k": (Hkv * 128, H), "v": (Hkv * 128, H),
                 "out": (H, Hq * 128), "gate": (F, H), "up": (F, H), "down": (H, F)}
        vi, seq, si = 1, V * H * 4, 0
        for l in range(L):
            for name in model_files.ORDER:
                if name.endswith("norm"):
                    n = F if name == "ffn_sub_norm" else H
                    nbytes = n * 4
                else:
                    N, K = sizes[name]
                    nbytes = N * K // 4
                off = views[vi] if vi < len(views) else seq
                vi += 1
                seq += nbytes
                which = WHICH[name]
                sc = ctypes.c_float()
                cnt = R.ref_engine_layer_data(e, l, which, None, None)
                buf = np.empty(cnt, np.int8 if which < 7 else np.float32)
                R.ref_engine_layer_data(e, l, which, buf.ctypes.data, ctypes.byref(sc))
                if which < 7:
                    if off + nbytes <= raw.size:
                        want = oracle.tl1_pack_raw(raw[off:off + nbytes].reshape(N // 4, K), N, K)
                    else:
                        want = np.full(N // 64 * K // 2 * 32, 0x55, np.uint8)
                    assert np.array_equal(buf.view(np.uint8), want), (l, name)
                    assert sc.value == (scales[si] if si < len(scales) else 1.0)
                    si += 1
                else:
                    if off + nbytes <= raw.size:
                        want = raw[off:off + nbytes].view(np.float32)
                    else:
                        want = np.ones(nbytes // 4, np.float32)
                    assert np.array_equal(buf, want), (l, name)
        codes = np.empty((V, H), np.int8)
        hs = np.empty(V, np.float32)
        fin = np.empty(H, np.float32)
        R.ref_engine_head_data(e, codes.ctypes.data, hs.ctypes.data, fin.ctypes.data)
        oc, os_ = oracle.quant_rows_i8(T["embed"])
        assert np.array_equal(codes, oc)
        assert np.array_equal(hs, os_)
        foff = views[vi] if vi < len(views) else seq
        want = (raw[foff:foff + H * 4].view(np.float32) if foff + H * 4 <= raw.size
                else np.ones(H, np.float32))
        assert np.array_equal(fin, want)
    finally:
        R.ref_engine_destroy(e)
