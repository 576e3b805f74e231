"""ctypes binding of the engine C API (include/tenzo.h plus the engine
extensions in include/tenzo_hip.h), mirroring the reference's C API
(``include/tenzo.h:92-193``, implemented at ``TenzoEngine.cpp:2086-2204``).

``Engine`` owns one ``tenzo_engine_t``; weights come from host numpy arrays in
the reference's formats (TL1 blocks, int8 LM head with per-row scales) and are
copied to the device when set. Every decode step runs on the GPU.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib, synth

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float


class Config(ctypes.Structure):
    """tenzo_config_t (reference include/tenzo.h:53-64)."""
    _fields_ = [("hidden_size", _I), ("num_q_heads", _I), ("num_kv_heads", _I),
                ("head_dim", _I), ("num_layers", _I), ("ffn_dim", _I), ("vocab_size", _I),
                ("max_seq_len", _I), ("kv_mode", ctypes.c_char_p), ("device", ctypes.c_char_p)]


class SamplingParams(ctypes.Structure):
    """tenzo_sampling_params_t (reference include/tenzo.h:66-72)."""
    _fields_ = [("temperature", _F), ("top_p", _F), ("top_k", _I),
                ("repetition_penalty", _F)]


class LayerWeights(ctypes.Structure):
    """tenzo_layer_weights_t (reference include/tenzo.h:75-87)."""
    _fields_ = [("q_w", _P), ("q_scale", _F), ("k_w", _P), ("k_scale", _F),
                ("v_w", _P), ("v_scale", _F), ("out_w", _P), ("out_scale", _F),
                ("gate_w", _P), ("gate_scale", _F), ("up_w", _P), ("up_scale", _F),
                ("down_w", _P), ("down_scale", _F),
                ("in_norm", _P), ("attn_sub_norm", _P), ("post_norm", _P),
                ("ffn_sub_norm", _P)]


def _sig(L):
    L.tenzo_default_config.restype = Config
    L.tenzo_default_config.argtypes = []
    L.tenzo_default_sampling_params.restype = SamplingParams
    L.tenzo_default_sampling_params.argtypes = []
    return L


def lib():
    return _sig(_lib.load())


def default_config() -> Config:
    return lib().tenzo_default_config()


def default_sampling_params() -> SamplingParams:
    return lib().tenzo_default_sampling_params()


def config_from(cfg: synth.DecodeConfig) -> Config:
    c = default_config()
    c.hidden_size, c.num_q_heads, c.num_kv_heads = cfg.hidden, cfg.n_q_heads, cfg.n_kv_heads
    c.head_dim, c.num_layers, c.ffn_dim = synth.HEAD_DIM, cfg.n_layers, cfg.ffn
    c.vocab_size, c.max_seq_len = cfg.vocab, cfg.max_seq
    c.kv_mode = b"int8_fused"
    c.device = b"rocm"
    return c


def _ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return ctypes.c_void_p(a.ctypes.data)


class Engine:
    """One device-resident decode engine."""

    def __init__(self, cfg: synth.DecodeConfig | Config, kv_mode: str | None = None):
        """kv_mode: "int8_fused" (default), "tl1_fused", "popcount_fused" or "paged_int8"."""
        self.L = lib()
        self.cfg = cfg if isinstance(cfg, Config) else config_from(cfg)
        if kv_mode is not None:
            self._kv_mode = kv_mode.encode()  # the config borrows the string
            self.cfg.kv_mode = self._kv_mode
        self.kv_mode = (self.cfg.kv_mode or b"int8_fused").decode()
        self.h = self.L.tenzo_create_engine(ctypes.byref(self.cfg))
        if not self.h:
            raise RuntimeError("tenzo_create_engine failed: " +
                               self.L.tenzo_hip_last_error().decode(errors="replace"))

    # -- lifecycle --
    def close(self):
        if self.h:
            self.L.tenzo_destroy_engine(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc, what):
        _lib.check(rc, what)

    # -- weights --
    def set_layer(self, l: int, lw: synth.LayerWeights, mlp: bool = True):
        w = LayerWeights()
        names = ["q", "k", "v", "out", "gate", "up", "down"]
        for p, f in zip(synth.PROJ, names):
            arr = lw.tl1[p] if (mlp or p not in ("gate", "up", "down")) else None
            setattr(w, f + "_w", _ptr(arr).value if arr is not None else None)
            setattr(w, f + "_scale", float(lw.scale[p]))
        for f in ["in_norm", "attn_sub_norm", "post_norm", "ffn_sub_norm"]:
            arr = getattr(lw, f)
            setattr(w, f, _ptr(arr).value if arr is not None else None)
        self._check(self.L.tenzo_set_layer_weights(self.h, l, ctypes.byref(w)),
                    "tenzo_set_layer_weights")

    def set_model(self, sm: synth.SynthModel, kv: bool = True):
        for l, lw in enumerate(sm.layers):
            self.set_layer(l, lw)
        self._check(self.L.tenzo_set_final_norm(self.h, _ptr(sm.final_norm)),
                    "tenzo_set_final_norm")
        c = sm.cfg
        self._check(self.L.tenzo_set_lm_head_i8(self.h, _ptr(sm.embed), _ptr(sm.embed_scales),
                                                c.vocab, c.hidden), "tenzo_set_lm_head_i8")
        if kv:
            self.set_kv_from(sm)
        self.set_rope_theta(c.theta)

    def load_model(self, weights_path: str, mlir_path: str):
        """tenzo_load_model: weights.bin + model.mlir as the reference's exporter
        writes them."""
        self._check(self.L.tenzo_load_model(self.h, weights_path.encode(), mlir_path.encode()),
                    "tenzo_load_model")

    def set_kv_from(self, sm: synth.SynthModel):
        n = sm.ctx
        if self.kv_mode == "paged_int8":
            self.set_kv(np.ascontiguousarray(sm.kc[:, :, :n]), np.ascontiguousarray(sm.vc[:, :, :n]),
                        np.ascontiguousarray(sm.ks[:, :, :n]), np.ascontiguousarray(sm.vs[:, :, :n]),
                        n)
            return
        if self.kv_mode != "int8_fused":
            if n:
                raise ValueError("the synthetic model's cache is INT8; use set_kv for "
                                 f"{self.kv_mode}")
            self.set_kv(np.zeros(1, np.uint8), np.zeros(1, np.uint8), np.zeros(1, np.float32),
                        np.zeros(1, np.float32), 0)
            return
        kc = np.ascontiguousarray(sm.kc[:, :, :n])
        vc = np.ascontiguousarray(sm.vc[:, :, :n])
        ks = np.ascontiguousarray(sm.ks[:, :, :n].astype(np.float16)).view(np.uint16)
        vs = np.ascontiguousarray(sm.vs[:, :, :n].astype(np.float16)).view(np.uint16)
        self.set_kv(kc, vc, ks, vs, n)

    def set_kv(self, kc, vc, ks, vs, seq_len: int):
        """Host arrays [L][Hkv][seq_len][128] int8 and [L][Hkv][seq_len] fp16 bits
        (int8_fused), or [L][Hkv][seq_len][32] uint8 and fp32 (ternary modes)."""
        self._check(self.L.tenzo_hip_engine_set_kv(self.h, _ptr(kc), _ptr(vc), _ptr(ks), _ptr(vs),
                                                   seq_len, 0), "engine_set_kv")

    def set_kv_device(self, kc_ptr, vc_ptr, ks_ptr, vs_ptr, seq_len: int):
        self._check(self.L.tenzo_hip_engine_set_kv(self.h, kc_ptr, vc_ptr, ks_ptr, vs_ptr,
                                                   seq_len, 1), "engine_set_kv")

    def get_kv(self, seq_len: int):
        """int8_fused: codes [L][Hkv][n][128] int8 and fp32 (from fp16) scales;
        ternary modes: rows [L][Hkv][n][32] uint8 and fp32 scales."""
        c = self.cfg
        shape = (c.num_layers, c.num_kv_heads, seq_len)
        if self.kv_mode == "paged_int8":
            kc = np.empty(shape + (128,), np.int8)
            vc = np.empty_like(kc)
            ks = np.empty(shape, np.float32)
            vs = np.empty_like(ks)
            self._check(self.L.tenzo_hip_engine_get_kv(self.h, _ptr(kc), _ptr(vc), _ptr(ks),
                                                       _ptr(vs), seq_len), "engine_get_kv")
            return kc, vc, ks, vs
        if self.kv_mode != "int8_fused":
            kb = np.empty(shape + (32,), np.uint8)
            vb = np.empty_like(kb)
            ks = np.empty(shape, np.float32)
            vs = np.empty_like(ks)
            self._check(self.L.tenzo_hip_engine_get_kv(self.h, _ptr(kb), _ptr(vb), _ptr(ks),
                                                       _ptr(vs), seq_len), "engine_get_kv")
            return kb, vb, ks, vs
        kc = np.empty(shape + (128,), np.int8)
        vc = np.empty_like(kc)
        ks = np.empty(shape, np.uint16)
        vs = np.empty_like(ks)
        self._check(self.L.tenzo_hip_engine_get_kv(self.h, _ptr(kc), _ptr(vc), _ptr(ks), _ptr(vs),
                                                   seq_len), "engine_get_kv")
        return kc, vc, ks.view(np.float16).astype(np.float32), vs.view(np.float16).astype(np.float32)

    def block_table(self) -> np.ndarray:
        """The paged_int8 sequence's block table (logical -> physical block)."""
        n = self.L.tenzo_hip_engine_block_table(self.h, None, 0)
        out = np.zeros(max(n, 1), np.int32)
        self._check(min(0, self.L.tenzo_hip_engine_block_table(self.h, _ptr(out), n)),
                    "engine_block_table")
        return out[:n]

    def set_rope_theta(self, theta: float):
        self._check(self.L.tenzo_hip_engine_set_rope_theta(self.h, theta), "set_rope_theta")

    def use_graph(self, on: bool):
        self._check(self.L.tenzo_hip_engine_use_graph(self.h, int(bool(on))), "use_graph")

    MODES = {"eager": 0, "graph": 1, "persistent": 2}

    def set_mode(self, mode: str):
        """'persistent' (default), 'graph' or 'eager'."""
        self._check(self.L.tenzo_hip_engine_set_mode(self.h, self.MODES[mode]), "set_mode")

    @property
    def mode(self) -> str:
        m = int(self.L.tenzo_hip_engine_get_mode(self.h))
        return {v: k for k, v in self.MODES.items()}[m]

    # -- decode --
    @property
    def seq_len(self) -> int:
        return int(self.L.tenzo_get_seq_len(self.h))

    def reset(self):
        self.L.tenzo_reset(self.h)

    def rewind(self, seq_len: int):
        self._check(self.L.tenzo_hip_engine_set_seq_len(self.h, int(seq_len)), "set_seq_len")

    def prefill(self, token: int):
        self._check(self.L.tenzo_prefill_token(self.h, int(token)), "tenzo_prefill_token")

    def prefill_batch(self, tokens, exact: bool = False):
        """All prompt tokens at once (tenzo_hip_engine_prefill): the state of
        one prefill() per token (bit for bit when exact)."""
        arr = np.ascontiguousarray(tokens, np.int32)
        self._check(self.L.tenzo_hip_engine_prefill(self.h, _ptr(arr), int(arr.size),
                                                    int(bool(exact))), "engine_prefill")

    def step(self, token: int, temperature: float = 0.0, penalty: float = 1.0,
             past=None, top_k: int = 40, top_p: float = 0.9) -> int:
        p = SamplingParams(temperature, top_p, top_k, penalty)
        past_arr = None if past is None else np.ascontiguousarray(past, np.int32)
        n = 0 if past_arr is None else past_arr.size
        tok = self.L.tenzo_generate_step(self.h, int(token), ctypes.byref(p), _ptr(past_arr), n)
        if tok < 0:
            raise RuntimeError("tenzo_generate_step failed: " +
                               self.L.tenzo_hip_last_error().decode(errors="replace"))
        return int(tok)

    def decode(self, token: int, n: int):
        """n greedy steps chained on the device; returns (tokens, ms of the n
        steps by HIP events on the engine stream)."""
        out = np.empty(n, np.int32)
        ms = ctypes.c_float(0.0)
        self._check(self.L.tenzo_hip_engine_decode(self.h, int(token), int(n), _ptr(out),
                                                   ctypes.byref(ms)), "engine_decode")
        return out, float(ms.value)

    def logits(self) -> np.ndarray:
        out = np.empty(self.cfg.vocab_size, np.float32)
        self._check(self.L.tenzo_hip_engine_get_logits(self.h, _ptr(out)), "get_logits")
        return out

    def buffer(self, name: str) -> np.ndarray:
        c = self.cfg
        n = max(c.vocab_size, 2 * c.ffn_dim, c.hidden_size + 2 * c.num_kv_heads * 128)
        out = np.empty(n, np.float32)
        self._check(self.L.tenzo_hip_engine_get_buffer(self.h, name.encode(), _ptr(out), n),
                    f"get_buffer({name})")
        sizes = {"x": c.hidden_size, "qkv": c.hidden_size + 2 * c.num_kv_heads * 128,
                 "attn_out": c.hidden_size, "h1": c.hidden_size, "gate_up": 2 * c.ffn_dim,
                 "logits": c.vocab_size}
        return out[:sizes[name]].copy()

    LAYER_STATE = {"x": (0, np.float32), "h1": (1, np.float32), "attn_out": (2, np.float32),
                   "acc_qkv": (3, np.int32), "acc_o": (4, np.int32), "acc_gu": (5, np.int32),
                   "acc_down": (6, np.int32)}

    def layer_state(self, layer: int, name: str) -> np.ndarray:
        """Layer `layer`'s state from the last persistent step: its input "x",
        "h1", "attn_out" (fp32), or the int32 TL1 sums sum_k (w_k + 1) a_k
        "acc_qkv", "acc_o", "acc_gu", "acc_down" (tenzo_hip_engine_get_layer_state)."""
        which, dt = self.LAYER_STATE[name]
        c = self.cfg
        n = max(2 * c.ffn_dim, c.hidden_size + 2 * c.num_kv_heads * 128,
                c.num_q_heads * 128 + 2 * c.num_kv_heads * 128)
        out = np.empty(n, dt)
        self._check(self.L.tenzo_hip_engine_get_layer_state(self.h, int(layer), which, _ptr(out), n),
                    f"get_layer_state({name})")
        q, kv, H, F = c.num_q_heads * 128, c.num_kv_heads * 128, c.hidden_size, c.ffn_dim
        size = {0: H, 1: H, 2: q, 3: q + 2 * kv, 4: H, 5: 2 * F, 6: H}[which]
        return out[:size].copy()

    def trace(self, on: bool = True):
        """Record per-stage barrier timestamps of the persistent kernel."""
        self._check(self.L.tenzo_hip_engine_trace(self.h, int(bool(on))), "engine_trace")

    def get_trace(self) -> np.ndarray:
        """[stages][nwg][2] wall-clock ticks (100 MHz): reach / leave the
        barrier after each stage, for the last step."""
        n = int(self.L.tenzo_hip_engine_get_trace(self.h, None, 0))
        if n < 0:
            raise RuntimeError("no trace (call trace(True) first)")
        out = np.empty(n, np.uint64)
        if self.L.tenzo_hip_engine_get_trace(self.h, _ptr(out), n) != n:
            raise RuntimeError("get_trace failed")
        stages = 5 * self.cfg.num_layers + 1
        return out.reshape(stages, -1, 2)

    def stream(self) -> int:
        return int(self.L.tenzo_hip_engine_stream(self.h) or 0)
