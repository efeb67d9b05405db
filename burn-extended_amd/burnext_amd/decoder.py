"""GPT-OSS decoder decode step around the MoE layer, over the C ABI (include/burnext_gptoss.h).

Reference surface (ariawisp/burn-extended):
  GptOssConfig                                   src/models/gpt_oss.rs:18-82
  GptOssConfig::init (random init)               src/models/gpt_oss.rs:115-189
  AutoregressiveModel::init_cache / forward_logits (decode branch)   src/models/gpt_oss.rs:199-252
  generate (greedy)                              src/generate/mod.rs:52-110, src/sampling/mod.rs:110-115
  WindowPolicy::EveryOther                       src/cache/mod.rs:7-44

Everything on the step runs in libburnext_moe.so (HIP, gfx950): dense projections, RoPE, the
rolling KV cache, sink attention, RmsNorms, the MoE layers and the greedy argmax.  This module
generates or takes the weights, creates the device objects and marshals calls.
"""
from __future__ import annotations

import ctypes
import dataclasses
import math

import numpy as np
import torch

from . import _native as N
from .moe import MoeLayer, _stream
from .synth import MoeLayerData, _rng, bf16_bits_to_f32, make_layer


@dataclasses.dataclass
class GptOssConfig:
    """Mirror of GptOssConfig (src/models/gpt_oss.rs:18-47) for the decode path.

    ``window_policy`` / ``window`` / ``full_on_even`` are WindowPolicy (Full, Fixed(window),
    EveryOther { window, full_on_even }); ``max_seq_len`` bounds the
    decode positions (the RoPE table length); ``sink_tokens`` (default 0, as the reference's
    default, src/models/gpt_oss.rs:70) keeps the first positions' cache rows through eviction and
    widens each window by that many rows (src/attention/streaming_mqa.rs:332-339).  Beyond the
    reference: ``rope_theta`` (the reference
    takes Burn's default base 10000; GPT-OSS uses 150000), ``rope_head_stride`` (1 = the
    reference's head-indexed RoPE positions, 0 = one position per token), ``scale_dk`` (scores
    divided by sqrt(scale_dk); 1 = pre-scaled q/k as the reference's GPT-OSS layers),
    ``kv_bf16`` (bf16 cache rows instead of the reference's f32) and ``experts_bf16`` (the expert
    projections on the normalised rows rounded to bf16 instead of f32)."""
    vocab_size: int = 201088
    d_model: int = 2880
    n_layers: int = 24
    n_heads: int = 64
    head_dim: int = 64
    kv_heads: int = 8
    ffn_hidden: int = 2880
    num_experts: int = 32
    experts_per_token: int = 4
    swiglu_alpha: float = 1.702
    swiglu_limit: float = 7.0
    cache_len: int = 8192
    window_policy: str = "every_other"  # WindowPolicy: "full", "fixed" (Fixed(window)), "every_other"
    window: int = 128
    full_on_even: bool = True
    max_seq_len: int = 8192
    learned_sinks: bool = True
    use_ntk_yarn: bool = True
    rope_theta: float = 150000.0
    rope_scaling_factor: float = 32.0
    rope_initial_context: float = 4096.0
    rope_ntk_alpha: float = 1.0
    rope_ntk_beta: float = 32.0
    rope_head_stride: int = 1
    scale_dk: float = 1.0
    rms_eps: float = 1e-5
    kv_bf16: bool = False
    sink_tokens: int = 0  # rows of the first positions the cache keeps through eviction (< cache_len)
    experts_bf16: bool = False  # expert projections on bf16-rounded rows (one MFMA term; not in the reference)

    @property
    def window_policy_code(self) -> int:
        return {"full": 0, "fixed": 1, "every_other": 2}[self.window_policy]

    def layer_window(self, layer: int, caller: int = 0) -> int:
        """WindowPolicy::window_for(layer) combined with the caller's window (0 = Full)."""
        pw = {"full": 0, "fixed": self.window,
              "every_other": 0 if (layer % 2 == 0) == self.full_on_even else self.window}[self.window_policy]
        if pw == 0:
            return caller
        return pw if caller == 0 else min(pw, caller)

    def c(self, max_batch: int) -> N.GptOssConfigC:
        yarn = self.use_ntk_yarn
        return N.GptOssConfigC(self.vocab_size, self.d_model, self.n_layers, self.n_heads, self.kv_heads,
                               self.head_dim, max_batch, self.cache_len, self.window_policy_code, self.window,
                               int(self.full_on_even),
                               int(self.rope_head_stride), self.max_seq_len, int(self.kv_bf16), self.rms_eps,
                               self.rope_theta, self.rope_scaling_factor if yarn else 1.0,
                               self.rope_initial_context, self.rope_ntk_alpha, self.rope_ntk_beta, self.scale_dk,
                               self.sink_tokens, int(self.experts_bf16))


GPT_OSS_20B = GptOssConfig()

# stream ids of the dense decoder tensors (disjoint from the MoE layer's: offset by 100)
_S_EMB, _S_NA, _S_WQ, _S_BQ, _S_WK, _S_BK, _S_WV, _S_BV, _S_WO, _S_BO, _S_SINK, _S_NF, _S_LM = range(100, 113)


def _bf16_bits_fast(a: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits (nearest-even) in 32-bit arithmetic: exact for finite inputs (the
    largest finite pattern plus 0x8000 stays below 2^32); the generator makes no NaN."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))) >> np.uint32(16)).astype(np.uint16)


def _uniform_bits(seed, stream, shape, bound, sub=0, chunk=1 << 24):
    """U(-bound, bound) float32 samples rounded to bf16 bits, generated in chunks."""
    g = _rng(seed, stream, sub)
    n = int(np.prod(shape))
    out = np.empty(n, np.uint16)
    for s in range(0, n, chunk):
        m = min(chunk, n - s)
        out[s:s + m] = _bf16_bits_fast(((g.random(m, dtype=np.float32) * 2.0 - 1.0) * bound).astype(np.float32))
    return out.reshape(shape)


def _normal_bits(seed, stream, shape, std=1.0, mean=0.0, sub=0, chunk=1 << 24):
    g = _rng(seed, stream, sub)
    n = int(np.prod(shape))
    out = np.empty(n, np.uint16)
    for s in range(0, n, chunk):
        m = min(chunk, n - s)
        out[s:s + m] = _bf16_bits_fast((g.standard_normal(m, dtype=np.float32) * std + mean).astype(np.float32))
    return out.reshape(shape)


@dataclasses.dataclass
class DecoderData:
    """Host weights of a decoder (bf16 bit patterns, Burn Linear weights transposed to [out, in],
    layer tensors stacked on a leading layer axis) and its MoE layers."""
    cfg: GptOssConfig
    tok_emb: np.ndarray     # [V, D]
    norm_attn: np.ndarray   # [L, D]
    wq: np.ndarray          # [L, nH dk, D]
    bq: np.ndarray          # [L, nH dk]
    wk: np.ndarray          # [L, kvH dk, D]
    bk: np.ndarray
    wv: np.ndarray
    bv: np.ndarray
    wo: np.ndarray          # [L, D, nH dk]
    bo: np.ndarray          # [L, D]
    sinks: np.ndarray | None  # [L, nH] (head h = kv head h // groups, group h % groups)
    norm_final: np.ndarray  # [D]
    lm_head: np.ndarray     # [V, D]
    moe: list[MoeLayerData]

    def f32(self, name: str) -> np.ndarray:
        return bf16_bits_to_f32(getattr(self, name))


def make_decoder(cfg: GptOssConfig, seed: int = 0, sinks_std: float = 0.0, norm_std: float = 0.0,
                 moe_dtype: str = "bf16") -> DecoderData:
    """Seeded random-init weights of the reference's shapes (GptOssConfig::init): Linear weights
    and biases U(+-1/sqrt(fan_in)) (KaimingUniform with gain 1/sqrt(3)), embedding N(0, 1),
    RmsNorm gammas 1 (N(1, norm_std) when norm_std > 0), sinks 0 (N(0, sinks_std) when
    sinks_std > 0), MoE layers as synth.make_layer with seed (seed, layer) and the decoder's own
    RmsNorm gamma folded in by the layer (with_gamma when norm_std > 0)."""
    D, L, V = cfg.d_model, cfg.n_layers, cfg.vocab_size
    qd, kd = cfg.n_heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    bd, bq = 1.0 / math.sqrt(D), 1.0 / math.sqrt(qd)
    ones = np.full(D, 0x3F80, np.uint16)
    gam = (lambda st, shape: _normal_bits(seed, st, shape, norm_std, 1.0)) if norm_std > 0 else \
        (lambda st, shape: np.broadcast_to(ones, shape).copy())
    data = DecoderData(
        cfg=cfg,
        tok_emb=_normal_bits(seed, _S_EMB, (V, D)),
        norm_attn=gam(_S_NA, (L, D)),
        wq=_uniform_bits(seed, _S_WQ, (L, qd, D), bd), bq=_uniform_bits(seed, _S_BQ, (L, qd), bd),
        wk=_uniform_bits(seed, _S_WK, (L, kd, D), bd), bk=_uniform_bits(seed, _S_BK, (L, kd), bd),
        wv=_uniform_bits(seed, _S_WV, (L, kd, D), bd), bv=_uniform_bits(seed, _S_BV, (L, kd), bd),
        wo=_uniform_bits(seed, _S_WO, (L, D, qd), bq), bo=_uniform_bits(seed, _S_BO, (L, D), bq),
        sinks=(None if not cfg.learned_sinks else
               (_normal_bits(seed, _S_SINK, (L, cfg.n_heads), sinks_std) if sinks_std > 0
                else np.zeros((L, cfg.n_heads), np.uint16))),
        norm_final=gam(_S_NF, (D,)),
        lm_head=_uniform_bits(seed, _S_LM, (V, D), bd),
        moe=[make_layer(D, cfg.ffn_hidden, cfg.num_experts, cfg.experts_per_token, seed=seed * 1000 + 1 + l,
                        dtype=moe_dtype, with_gamma=norm_std > 0) for l in range(L)],
    )
    for m in data.moe:
        m.swiglu_alpha, m.swiglu_limit, m.rms_eps = cfg.swiglu_alpha, cfg.swiglu_limit, cfg.rms_eps
    return data


def _ptr(a):
    return None if a is None else np.ascontiguousarray(a).ctypes.data_as(ctypes.c_void_p)


class GptOssDecoder:
    """Device-resident decoder (burnext_gptoss_create) with its MoE layers and KV cache.

    decode() is one AutoregressiveModel::forward_logits decode call plus greedy sampling; the
    cache position bookkeeping is the library's (reset() empties the cache)."""

    def __init__(self, data: DecoderData, max_batch: int, device: int = 0, moe_layers: list[MoeLayer] | None = None):
        cfg = data.cfg
        self.cfg, self.device, self.max_batch = cfg, device, max_batch
        self.moe_layers = moe_layers or [MoeLayer(m, device=device) for m in data.moe]
        handles = (ctypes.c_void_p * cfg.n_layers)(*[m.handle.value for m in self.moe_layers])
        arrs = {k: np.ascontiguousarray(getattr(data, k)) for k in
                ("tok_emb", "norm_attn", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "norm_final", "lm_head")}
        sinks = None if data.sinks is None else np.ascontiguousarray(data.sinks)
        w = N.GptOssWeightsC(*[_ptr(arrs[k]) for k in ("tok_emb", "norm_attn", "wq", "bq", "wk", "bk", "wv", "bv",
                                                        "wo", "bo")], _ptr(sinks), _ptr(arrs["norm_final"]),
                             _ptr(arrs["lm_head"]))
        c = cfg.c(max_batch)
        h = ctypes.c_void_p()
        N.check(N.lib().burnext_gptoss_create(ctypes.byref(c), ctypes.byref(w), handles, device, ctypes.byref(h)))
        self.handle = h
        self._ws = None

    def close(self) -> None:
        if getattr(self, "handle", None) is not None and self.handle.value:
            N.lib().burnext_gptoss_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def workspace_size(self, batch: int) -> int:
        b = ctypes.c_uint64()
        N.check(N.lib().burnext_gptoss_workspace_size(self.handle, batch, ctypes.byref(b)))
        return b.value

    def workspace(self, batch: int) -> torch.Tensor:
        need = self.workspace_size(batch)
        if self._ws is None or self._ws[1] < need:
            raw = torch.empty(need + 256, dtype=torch.uint8, device=f"cuda:{self.device}")
            self._ws = (raw, need, (-raw.data_ptr()) % 256)
        raw, _, off = self._ws
        return raw[off:off + need]

    def reset(self) -> None:
        N.check(N.lib().burnext_gptoss_reset(self.handle))

    def cache_load(self, k: torch.Tensor, v: torch.Tensor, stream=None) -> None:
        """Cache rows for positions 0 .. len-1: k, v f32 [L, B, len, kvH, dk] on the device."""
        assert k.dtype == torch.float32 and v.dtype == torch.float32 and k.is_contiguous() and v.is_contiguous()
        L, B, ln, H, dk = k.shape
        assert (L, H, dk) == (self.cfg.n_layers, self.cfg.kv_heads, self.cfg.head_dim) and v.shape == k.shape
        N.check(N.lib().burnext_gptoss_cache_load(self.handle, ctypes.c_void_p(k.data_ptr()),
                                                  ctypes.c_void_p(v.data_ptr()), B, ln, _stream(stream)))

    def decode(self, tokens: torch.Tensor, pos: int, logits: bool = False, hidden: bool = False, window: int = 0,
               out: torch.Tensor | None = None, workspace: torch.Tensor | None = None, stream=None):
        """One decode step: tokens int32 [B] (device) at absolute position pos, `window` the caller's
        AttnWindow (0 = Full).  Returns next tokens int32 [B] (and the logits [B, V] / final hidden
        [B, D] when asked)."""
        assert tokens.is_cuda and tokens.dtype == torch.int32 and tokens.dim() == 1
        B = tokens.shape[0]
        nxt = torch.empty(B, dtype=torch.int32, device=tokens.device) if out is None else out
        lg = torch.empty((B, self.cfg.vocab_size), dtype=torch.float32, device=tokens.device) if logits else None
        hd = torch.empty((B, self.cfg.d_model), dtype=torch.float32, device=tokens.device) if hidden else None
        ws = self.workspace(B) if workspace is None else workspace
        N.check(N.lib().burnext_gptoss_decode(
            self.handle, ctypes.c_void_p(tokens.data_ptr()), B, pos, window, ctypes.c_void_p(nxt.data_ptr()),
            None if lg is None else ctypes.c_void_p(lg.data_ptr()),
            None if hd is None else ctypes.c_void_p(hd.data_ptr()), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
            _stream(stream)))
        if logits or hidden:
            return (nxt,) + ((lg,) if logits else ()) + ((hd,) if hidden else ())
        return nxt

    def generate(self, first: torch.Tensor, start_pos: int, steps: int, window: int = 0) -> torch.Tensor:
        """Greedy decode of `steps` tokens after `first` [B] at start_pos (src/generate/mod.rs:52-110
        with temperature 0): returns [B, steps] int32."""
        outs = []
        tok = first
        for s in range(steps):
            tok = self.decode(tok, start_pos + s, window=window)
            outs.append(tok)
        return torch.stack(outs, dim=1)
