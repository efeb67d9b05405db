"""ctypes front-end of the CPU oracle (oracle/moe_oracle.c, oracle/decoder_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() (as the checker) and
bench.py's cpu_baseline leg.  The product library never loads it.
"""
from __future__ import annotations

import ctypes

import pathlib
import subprocess

import numpy as np

_HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = _HERE / "_build" / "libmoe_oracle.so"
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64 = ctypes.c_int64


class _Cfg(ctypes.Structure):
    _fields_ = [("d", ctypes.c_int64), ("f", ctypes.c_int64), ("e", ctypes.c_int64), ("k", ctypes.c_int64),
                ("alpha", ctypes.c_float), ("limit", ctypes.c_float), ("eps", ctypes.c_float),
                ("bf16_rows", ctypes.c_int64)]


class _DecCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in ("vocab", "d_model", "n_layers", "n_heads", "kv_heads", "head_dim",
                                              "batch", "cache_len", "window_policy", "window", "full_on_even",
                                              "rope_head_stride")] + \
               [("rms_eps", ctypes.c_float), ("scale_dk", ctypes.c_float), ("sink_tokens", ctypes.c_int64),
                ("experts_bf16", ctypes.c_int64)]


class _DecWeights(ctypes.Structure):
    _fields_ = [(n, _f32p) for n in ("tok_emb", "norm_attn", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "sinks",
                                     "norm_final", "lm_head", "rope_table")]


class _MoeLayerC(ctypes.Structure):
    _fields_ = [("cfg", _Cfg), ("w1b", _u8p), ("w1s", _u8p), ("w2b", _u8p), ("w2s", _u8p), ("ue8_offset", ctypes.c_int),
                ("b1", _f32p), ("b2", _f32p), ("router_w", _f32p), ("router_b", _f32p), ("gamma", _f32p),
                ("layout", ctypes.c_int)]


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.oracle_fp4_value.restype = ctypes.c_float
        L.oracle_fp4_value.argtypes = [ctypes.c_int]
        L.oracle_e8m0_scale.restype = ctypes.c_float
        L.oracle_e8m0_scale.argtypes = [ctypes.c_int]
        L.oracle_dequant_mxfp4_bytes.argtypes = [_u8p, _u8p, _i64, _i64, _f32p]
        L.oracle_dequant_matrix.argtypes = [_u8p, _u8p, _i64, _i64, _i64, _i64, ctypes.c_int, _f32p]
        L.oracle_rmsnorm.argtypes = [_f32p, _i64, _i64, _f32p, ctypes.c_float, _f32p]
        L.oracle_router.argtypes = [_f32p, _i64, _i64, _f32p, _f32p, _i64, _f32p]
        L.oracle_route_logits.argtypes = [_f32p, _i64, _i64, _f32p, ctypes.c_float, ctypes.c_int, _f32p, _f32p,
                                          _i64, _f32p]
        L.oracle_topk_softmax.argtypes = [_f32p, _i64, _i64, _i64, _i32p, _f32p]
        L.oracle_dispatch.argtypes = [_i32p, _i64, _i64, _i64, _i32p, _i32p, _i32p]
        L.oracle_swiglu.restype = ctypes.c_float
        L.oracle_swiglu.argtypes = [ctypes.c_float] * 4
        L.oracle_round_bf16.restype = ctypes.c_float
        L.oracle_round_bf16.argtypes = [ctypes.c_float]
        fwd = [_f32p, _i64, ctypes.POINTER(_Cfg), _u8p, _u8p, _u8p, _u8p, ctypes.c_int, _f32p, _f32p, _f32p,
               _f32p, _f32p]
        L.oracle_moe_forward.argtypes = fwd + [ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _i32p, _f32p]
        L.oracle_moe_forward.restype = ctypes.c_int
        L.oracle_moe_forward_reference.argtypes = fwd + [ctypes.c_int, _f32p]
        L.oracle_moe_forward_reference.restype = ctypes.c_int
        L.oracle_num_threads.restype = ctypes.c_int
        L.oracle_yarn_inv_freq.restype = ctypes.c_int
        L.oracle_yarn_inv_freq.argtypes = [_i64] + [ctypes.c_double] * 5 + [_f32p, _f32p]
        L.oracle_rope_table.argtypes = [_f32p, _i64, ctypes.c_float, _i64, _f32p]
        L.oracle_rope_apply.argtypes = [_f32p, _i64, _i64, _i64, _i64, _f32p]
        L.oracle_linear.argtypes = [_f32p, _i64, _i64, _f32p, _f32p, _i64, _f32p]
        L.oracle_sink_attention.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64, _f32p,
                                            ctypes.c_float, _f32p]
        L.oracle_decoder_step.restype = ctypes.c_int
        L.oracle_decoder_step.argtypes = [ctypes.POINTER(_DecCfg), ctypes.POINTER(_DecWeights),
                                          ctypes.POINTER(_MoeLayerC), _i32p, _i64, _i64, _f32p, _f32p,
                                          ctypes.POINTER(_i64), _f32p, _f32p, _i32p]
        _lib = L
    return _lib


def _p(a, t):
    return a.ctypes.data_as(t) if a is not None else None


def _c(a, dt):
    return None if a is None else np.ascontiguousarray(a, dtype=dt)


def fp4_value(nib: int) -> float:
    return lib().oracle_fp4_value(nib)


def e8m0_scale(s: int) -> float:
    return lib().oracle_e8m0_scale(s)


def dequant_mxfp4_bytes(blocks, blocks_shape, scales, scales_shape) -> np.ndarray:
    """Signature of the reference test helper (src/loader/mxfp4.rs:56-79)."""
    rows = int(np.prod(scales_shape)) if len(scales_shape) else 1
    b = int(blocks_shape[-1])
    bl = _c(np.asarray(blocks, np.uint8).reshape(-1), np.uint8)
    sc = _c(np.asarray(scales, np.uint8).reshape(-1), np.uint8)
    assert bl.size == rows * b and sc.size == rows
    out = np.empty(rows * 2 * b, np.float32)
    lib().oracle_dequant_mxfp4_bytes(_p(bl, _u8p), _p(sc, _u8p), rows, b, _p(out, _f32p))
    return out


def dequant_matrix(blocks, scales, rows, cols, ue8_offset=0) -> np.ndarray:
    bpr, gpr = (cols + 1) // 2, (cols + 31) // 32
    bl = _c(blocks, np.uint8).reshape(-1)
    sc = _c(scales, np.uint8).reshape(-1)
    assert bl.size == rows * bpr and sc.size == rows * gpr
    out = np.empty((rows, cols), np.float32)
    lib().oracle_dequant_matrix(_p(bl, _u8p), _p(sc, _u8p), rows, cols, bpr, gpr, ue8_offset, _p(out, _f32p))
    return out


def rmsnorm(x, gamma=None, eps=1e-5) -> np.ndarray:
    x = _c(x, np.float32)
    n, d = x.shape
    g = _c(gamma, np.float32)
    out = np.empty_like(x)
    lib().oracle_rmsnorm(_p(x, _f32p), n, d, _p(g, _f32p), eps, _p(out, _f32p))
    return out


def router(xn, w, b=None) -> np.ndarray:
    xn, w, b = _c(xn, np.float32), _c(w, np.float32), _c(b, np.float32)
    n, d = xn.shape
    e = w.shape[0]
    out = np.empty((n, e), np.float32)
    lib().oracle_router(_p(xn, _f32p), n, d, _p(w, _f32p), _p(b, _f32p), e, _p(out, _f32p))
    return out


def route_logits(x, w, b=None, gamma=None, eps=1e-5, apply_rmsnorm=True) -> np.ndarray:
    """Router logits in the GPU router's order (see oracle_route_logits)."""
    x, w, b, g = _c(x, np.float32), _c(w, np.float32), _c(b, np.float32), _c(gamma, np.float32)
    n, d = x.shape
    e = w.shape[0]
    out = np.empty((n, e), np.float32)
    lib().oracle_route_logits(_p(x, _f32p), n, d, _p(g, _f32p), eps, int(apply_rmsnorm), _p(w, _f32p),
                              _p(b, _f32p), e, _p(out, _f32p))
    return out


def topk_softmax(logits, k):
    lg = _c(logits, np.float32)
    n, e = lg.shape
    kk = min(max(int(k), 1), e)
    idx = np.empty((n, kk), np.int32)
    w = np.empty((n, kk), np.float32)
    lib().oracle_topk_softmax(_p(lg, _f32p), n, e, kk, _p(idx, _i32p), _p(w, _f32p))
    return idx, w


def dispatch(idx, num_experts):
    idx = _c(idx, np.int32)
    n, k = idx.shape
    seg = np.empty(num_experts + 1, np.int32)
    perm = np.empty(n * k, np.int32)
    pos = np.empty(n * k, np.int32)
    lib().oracle_dispatch(_p(idx, _i32p), n, k, num_experts, _p(seg, _i32p), _p(perm, _i32p), _p(pos, _i32p))
    return seg, perm, pos


def swiglu(g, l, alpha=1.702, limit=7.0) -> float:
    return lib().oracle_swiglu(g, l, alpha, limit)


def _layer_args(layer):
    cfg = _Cfg(layer.d_model, layer.ffn_hidden, layer.num_experts, layer.experts_per_token, layer.swiglu_alpha,
               layer.swiglu_limit, layer.rms_eps)
    arrs = dict(w1b=_c(layer.w1_blocks, np.uint8), w1s=_c(layer.w1_scales, np.uint8),
                w2b=_c(layer.w2_blocks, np.uint8), w2s=_c(layer.w2_scales, np.uint8),
                b1=_c(layer.b1_f32, np.float32), b2=_c(layer.b2_f32, np.float32),
                rw=_c(layer.router_w_f32, np.float32), rb=_c(layer.router_b_f32, np.float32),
                g=_c(layer.gamma_f32, np.float32))
    return cfg, arrs


def moe_forward(layer, x, apply_rmsnorm=True, add_residual=True, layout=None, bf16_rows=False):
    """The build's layer semantics (see oracle_moe_forward).  Returns (y, idx, w).  bf16_rows:
    the expert products on rows and SwiGLU outputs rounded to bf16 (the device's one-term option)."""
    x = _c(x, np.float32)
    n, d = x.shape
    assert d == layer.d_model
    cfg, a = _layer_args(layer)
    cfg.bf16_rows = int(bf16_rows)
    kk = min(max(layer.experts_per_token, 1), layer.num_experts)
    lay = {"halves": 0, "interleaved": 1}[layout or layer.gate_up_layout]
    y = np.empty_like(x)
    idx = np.empty((n, kk), np.int32)
    w = np.empty((n, kk), np.float32)
    rc = lib().oracle_moe_forward(_p(x, _f32p), n, ctypes.byref(cfg), _p(a["w1b"], _u8p), _p(a["w1s"], _u8p),
                                  _p(a["w2b"], _u8p), _p(a["w2s"], _u8p), layer.ue8_offset, _p(a["b1"], _f32p),
                                  _p(a["b2"], _f32p), _p(a["rw"], _f32p), _p(a["rb"], _f32p), _p(a["g"], _f32p),
                                  lay, int(apply_rmsnorm), int(add_residual), _p(y, _f32p), _p(idx, _i32p),
                                  _p(w, _f32p))
    assert rc == 0
    return y, idx, w


def moe_forward_reference(layer, x, b2_per_ftile=True):
    """Literal reference algorithm (halves pairing, dense W1, b2 per f-tile unless b2_per_ftile is
    False), OpenMP-parallel."""
    x = _c(x, np.float32)
    n, d = x.shape
    cfg, a = _layer_args(layer)
    y = np.empty_like(x)
    rc = lib().oracle_moe_forward_reference(_p(x, _f32p), n, ctypes.byref(cfg), _p(a["w1b"], _u8p),
                                            _p(a["w1s"], _u8p), _p(a["w2b"], _u8p), _p(a["w2s"], _u8p),
                                            layer.ue8_offset, _p(a["b1"], _f32p), _p(a["b2"], _f32p),
                                            _p(a["rw"], _f32p), _p(a["rb"], _f32p), _p(a["g"], _f32p),
                                            int(b2_per_ftile), _p(y, _f32p))
    assert rc == 0
    return y


# ---- decoder (oracle/decoder_oracle.c) ------------------------------------------------------------

def yarn_inv_freq(d, theta, factor=1.0, ctx=4096.0, alpha=1.0, beta=32.0):
    """(inv_freq [d/2] float32, concentration); raises ValueError where the reference asserts."""
    inv = np.empty(d // 2, np.float32)
    conc = ctypes.c_float()
    rc = lib().oracle_yarn_inv_freq(d, theta, factor, ctx, alpha, beta, _p(inv, _f32p), ctypes.byref(conc))
    if rc != 0:
        raise ValueError("YaRN thresholds out of range")
    return inv, conc.value


def rope_table(inv, d, conc, npos) -> np.ndarray:
    inv = _c(inv, np.float32)
    out = np.empty((npos, d // 2, 2), np.float32)
    lib().oracle_rope_table(_p(inv, _f32p), d, conc, npos, _p(out, _f32p))
    return out


def rope_apply(x, pos0, head_stride, table) -> np.ndarray:
    """x [heads, d] rotated (copy): head h at position pos0 + h * head_stride."""
    y = _c(x, np.float32).copy()
    heads, d = y.shape
    t = _c(table, np.float32)
    assert pos0 + (heads - 1) * head_stride < t.shape[0]
    lib().oracle_rope_apply(_p(y, _f32p), heads, d, pos0, head_stride, _p(t, _f32p))
    return y


def linear(x, w, bias=None) -> np.ndarray:
    x, w, b = _c(x, np.float32), _c(w, np.float32), _c(bias, np.float32)
    nb, k = x.shape
    n = w.shape[0]
    y = np.empty((nb, n), np.float32)
    lib().oracle_linear(_p(x, _f32p), nb, k, _p(w, _f32p), _p(b, _f32p), n, _p(y, _f32p))
    return y


def sink_attention(q, k, v, n_kv_heads, sinks=None, scale_dk=1.0) -> np.ndarray:
    """q [nh, d]; k, v [nk, n_kv_heads, d]; sinks [nh] or None -> [nh, d]."""
    q, k, v, s = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32), _c(sinks, np.float32)
    nh, d = q.shape
    nk = k.shape[0]
    out = np.empty((nh, d), np.float32)
    lib().oracle_sink_attention(_p(q, _f32p), _p(k, _f32p), _p(v, _f32p), nk, n_kv_heads * d, nh, n_kv_heads, d,
                                _p(s, _f32p), scale_dk, _p(out, _f32p))
    return out


class DecoderOracle:
    """CPU decoder state (f32 weights and cache) driven step by step by oracle_decoder_step.

    ``data`` is a burnext_amd.decoder.DecoderData; the cache is [L][B][cache_len][kvH][dk] f32.
    ``experts_bf16`` (default: the config's) models the device's bf16 expert rows."""

    def __init__(self, data, batch: int, experts_bf16=None):
        cfg = data.cfg
        self.cfg, self.batch = cfg, batch
        self.w = {k: np.ascontiguousarray(data.f32(k)) for k in
                  ("tok_emb", "norm_attn", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "norm_final", "lm_head")}
        self.w["sinks"] = None if data.sinks is None else np.ascontiguousarray(data.f32("sinks"))
        factor = cfg.rope_scaling_factor if cfg.use_ntk_yarn else 1.0
        inv, conc = yarn_inv_freq(cfg.head_dim, cfg.rope_theta, factor, cfg.rope_initial_context, cfg.rope_ntk_alpha,
                                  cfg.rope_ntk_beta)
        self.inv, self.conc = inv, conc
        self.table = rope_table(inv, cfg.head_dim, conc, cfg.max_seq_len + cfg.n_heads)
        shape = (cfg.n_layers, batch, cfg.cache_len, cfg.kv_heads, cfg.head_dim)
        self.k = np.zeros(shape, np.float32)
        self.v = np.zeros(shape, np.float32)
        self.used = 0
        self._moe = []
        self._keep = []
        for m in data.moe:
            c, a = _layer_args(m)
            self._keep.append(a)
            lay = {"halves": 0, "interleaved": 1}[m.gate_up_layout]
            self._moe.append(_MoeLayerC(c, _p(a["w1b"], _u8p), _p(a["w1s"], _u8p), _p(a["w2b"], _u8p),
                                        _p(a["w2s"], _u8p), m.ue8_offset, _p(a["b1"], _f32p), _p(a["b2"], _f32p),
                                        _p(a["rw"], _f32p), _p(a["rb"], _f32p), _p(a["g"], _f32p), lay))
        self._moe_arr = (_MoeLayerC * len(self._moe))(*self._moe)
        W = self.w
        self._wc = _DecWeights(*[_p(W[k], _f32p) for k in ("tok_emb", "norm_attn", "wq", "bq", "wk", "bk", "wv", "bv",
                                                           "wo", "bo", "sinks", "norm_final", "lm_head")],
                               _p(self.table, _f32p))
        self._cc = _DecCfg(cfg.vocab_size, cfg.d_model, cfg.n_layers, cfg.n_heads, cfg.kv_heads, cfg.head_dim, batch,
                           cfg.cache_len, cfg.window_policy_code, cfg.window, int(cfg.full_on_even),
                           cfg.rope_head_stride, cfg.rms_eps, cfg.scale_dk, cfg.sink_tokens,
                           int(cfg.experts_bf16 if experts_bf16 is None else experts_bf16))

    def load(self, k, v) -> None:
        """Cache rows for positions 0 .. len-1 (k, v [L, B, len, kvH, dk])."""
        ln = k.shape[2]
        self.k[:, :, :ln] = k
        self.v[:, :, :ln] = v
        self.used = ln

    def step(self, tokens, pos, window: int = 0):
        """One decode step (window: the caller's AttnWindow, 0 = Full): (next_tokens [B] int32,
        logits [B, V], hidden [B, D])."""
        cfg = self.cfg
        tok = _c(tokens, np.int32)
        assert tok.shape == (self.batch,)
        logits = np.empty((self.batch, cfg.vocab_size), np.float32)
        hidden = np.empty((self.batch, cfg.d_model), np.float32)
        nxt = np.empty(self.batch, np.int32)
        used = _i64(self.used)
        rc = lib().oracle_decoder_step(ctypes.byref(self._cc), ctypes.byref(self._wc), self._moe_arr, _p(tok, _i32p),
                                       pos, window, _p(self.k, _f32p), _p(self.v, _f32p), ctypes.byref(used),
                                       _p(logits, _f32p), _p(hidden, _f32p), _p(nxt, _i32p))
        assert rc == 0
        self.used = used.value
        return nxt, logits, hidden


def num_threads() -> int:
    return lib().oracle_num_threads()


def max_abs_rel(y, ref) -> float:
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(y - ref)) / (den if den > 0 else 1.0))


__all__ = [n for n in dir() if not n.startswith("_")]

