"""Seeded synthetic MoE layers and activations for the GPT-OSS shapes of the benchmark configs.

Every tensor has its own PCG64 stream derived from (master seed, stream id), so a tensor does not
change when another tensor's shape changes.  The distributions follow the benchmark description:

* activations ~ N(0, 1); router weight ~ N(0, 0.02); router bias 0 (or a Zipf popularity bias);
* expert weights are MXFP4: packed e2m1 bytes uniform over 0..255 (both nibbles uniform over the
  16 codes), e8m0 scale bytes uniform in 127-8 .. 127-4, stored with ``ue8_offset`` added mod 256
  as the model.bin exporter writes them (reference src/bin/gptoss_export.rs:529,562);
* expert biases ~ N(0, 0.01).

bf16 tensors are produced by rounding float32 samples to nearest-even and are returned both as
raw uint16 bits (what the device receives) and as the exactly equal float32 values.
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

# stream ids (stable: never renumber)
_S_X, _S_RW, _S_RB, _S_W1B, _S_W1S, _S_W2B, _S_W2S, _S_B1, _S_B2, _S_GAMMA, _S_ZIPF = range(11)


def _rng(seed: int, stream: int, sub: int = 0) -> np.random.Generator:
    return np.random.default_rng(np.random.SeedSequence([int(seed), int(stream), int(sub)]))


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (nearest-even), returning the uint16 bit patterns."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        r[nan] = 0x7FC0
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(a: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


@dataclasses.dataclass
class MoeLayerData:
    """Host-side tensors of one MoE layer in the reference's resident/on-disk form.

    w1_* is [E, 2F, bpr|gpr] (rows ordered by ``gate_up_layout``), w2_* is [E, D, bpr|gpr],
    biases [E, 2F] / [E, D] in the same row order, router weight [E, D] and bias [E].
    ``*_f32`` hold float values; ``*_bits`` the bf16 bit patterns when the dtype is bf16.
    """

    d_model: int
    ffn_hidden: int
    num_experts: int
    experts_per_token: int
    w1_blocks: np.ndarray
    w1_scales: np.ndarray
    w2_blocks: np.ndarray
    w2_scales: np.ndarray
    b1_f32: np.ndarray
    b2_f32: np.ndarray
    router_w_f32: np.ndarray
    router_b_f32: np.ndarray
    dtype: str  # "f32" or "bf16" for biases / router weight
    ue8_offset: int = 0
    gate_up_layout: str = "interleaved"
    swiglu_alpha: float = 1.702
    swiglu_limit: float = 7.0
    rms_eps: float = 1e-5
    gamma_f32: np.ndarray | None = None

    @property
    def b1_bits(self) -> np.ndarray:
        return f32_to_bf16_bits(self.b1_f32)

    @property
    def b2_bits(self) -> np.ndarray:
        return f32_to_bf16_bits(self.b2_f32)

    @property
    def router_w_bits(self) -> np.ndarray:
        return f32_to_bf16_bits(self.router_w_f32)

    @property
    def router_b_bits(self) -> np.ndarray:
        return f32_to_bf16_bits(self.router_b_f32)

    def expert_bytes(self) -> int:
        """HBM bytes of one expert: W1+W2 blocks and scales plus both biases (at `dtype`)."""
        D, F = self.d_model, self.ffn_hidden
        sb = 2 if self.dtype == "bf16" else 4
        return (2 * F * ((D + 1) // 2) + 2 * F * ((D + 31) // 32) + D * ((F + 1) // 2)
                + D * ((F + 31) // 32) + (2 * F + D) * sb)


def make_layer(d_model: int, ffn_hidden: int, num_experts: int, experts_per_token: int, seed: int = 0,
               dtype: str = "bf16", ue8_offset: int = 0, gate_up_layout: str = "interleaved",
               router_bias: np.ndarray | None = None, scale_lo: int = 127 - 8, scale_hi: int = 127 - 4,
               with_gamma: bool = False) -> MoeLayerData:
    D, F, E = int(d_model), int(ffn_hidden), int(num_experts)
    bpr1, gpr1 = (D + 1) // 2, (D + 31) // 32
    bpr2, gpr2 = (F + 1) // 2, (F + 31) // 32
    w1b = _rng(seed, _S_W1B).integers(0, 256, size=(E, 2 * F, bpr1), dtype=np.uint8)
    w1s = _rng(seed, _S_W1S).integers(scale_lo, scale_hi + 1, size=(E, 2 * F, gpr1), dtype=np.uint8)
    w2b = _rng(seed, _S_W2B).integers(0, 256, size=(E, D, bpr2), dtype=np.uint8)
    w2s = _rng(seed, _S_W2S).integers(scale_lo, scale_hi + 1, size=(E, D, gpr2), dtype=np.uint8)
    if ue8_offset:
        w1s = ((w1s.astype(np.int32) + ue8_offset) & 255).astype(np.uint8)
        w2s = ((w2s.astype(np.int32) + ue8_offset) & 255).astype(np.uint8)
    b1 = _rng(seed, _S_B1).normal(0.0, 0.01, size=(E, 2 * F)).astype(np.float32)
    b2 = _rng(seed, _S_B2).normal(0.0, 0.01, size=(E, D)).astype(np.float32)
    rw = _rng(seed, _S_RW).normal(0.0, 0.02, size=(E, D)).astype(np.float32)
    rb = np.zeros(E, np.float32) if router_bias is None else np.asarray(router_bias, np.float32).copy()
    gamma = None
    if with_gamma:
        gamma = _rng(seed, _S_GAMMA).normal(1.0, 0.1, size=(D,)).astype(np.float32)
    if dtype == "bf16":
        b1, b2, rw, rb = round_bf16(b1), round_bf16(b2), round_bf16(rw), round_bf16(rb)
        if gamma is not None:
            gamma = round_bf16(gamma)
    elif dtype != "f32":
        raise ValueError(dtype)
    return MoeLayerData(D, F, E, int(experts_per_token), w1b, w1s, w2b, w2s, b1, b2, rw, rb, dtype,
                        ue8_offset=ue8_offset, gate_up_layout=gate_up_layout, gamma_f32=gamma)


def make_tokens(n_tokens: int, d_model: int, seed: int = 0, dtype: str = "bf16", sub: int = 0) -> np.ndarray:
    """Activations ~N(0,1) as float32 (bf16-representable when dtype == 'bf16')."""
    x = _rng(seed, _S_X, sub).standard_normal(size=(int(n_tokens), int(d_model))).astype(np.float32)
    return round_bf16(x) if dtype == "bf16" else x


def zipf_router_bias(num_experts: int, s: float = 1.1, gamma: float = 1.0, seed: int = 0) -> np.ndarray:
    """Router bias b_e = -s * ln(r_e) * gamma, r a seeded permutation of 1..E.

    Expert popularity then decays with rank roughly like a Zipf law of exponent s.  ``gamma``
    sets how strongly the bias dominates the N(0, ~1) router logits.
    """
    r = _rng(seed, _S_ZIPF).permutation(num_experts) + 1
    return (-s * np.log(r.astype(np.float64)) * gamma).astype(np.float32)


# gamma of the C3 prefill router bias: calibrate_zipf_gamma() on the benchmark's seed-0 layer and
# tokens (T = 4096, D = 2880, E = 32, k = 4).  Realised routed entries by popularity rank: 2764,
# 2054, 1514, ..., 100, 98 against the ideal s = 1.1 shares 4096 (capped: a token takes an expert
# once), 2168, 1388, ..., 106, 102.
ZIPF_GAMMA_C3 = 0.70


def zipf_rank_counts_from_idx(idx: np.ndarray, num_experts: int, seed: int = 0) -> np.ndarray:
    """Routed entries per expert of a top-k index array, listed by the expert's Zipf popularity
    rank 1..E of zipf_router_bias(seed)."""
    c = np.bincount(np.asarray(idx).ravel(), minlength=num_experts)
    rank = _rng(seed, _S_ZIPF).permutation(num_experts)
    out = np.zeros(num_experts, np.int64)
    out[rank] = c
    return out


def zipf_rank_counts(logits: np.ndarray, k: int, num_experts: int, seed: int = 0) -> np.ndarray:
    """zipf_rank_counts_from_idx of the top-k (largest first, ties to the lower index) of each row
    of ``logits``."""
    return zipf_rank_counts_from_idx(np.argsort(-logits, axis=1, kind="stable")[:, :k], num_experts, seed)


def zipf_ideal_counts(num_experts: int, s: float, tokens: int, k: int) -> np.ndarray:
    """Ideal routed entries by rank: tokens * k * r^-s / H, capped at `tokens` (an expert is taken at
    most once per token)."""
    r = np.arange(1, num_experts + 1, dtype=np.float64)
    p = r ** -s / np.sum(r ** -s)
    return np.minimum(p * tokens * k, tokens)


def calibrate_zipf_gamma(layer: MoeLayerData, x: np.ndarray, s: float = 1.1, seed: int = 0,
                         grid=np.arange(0.30, 2.001, 0.05)) -> tuple[float, np.ndarray]:
    """The gamma of zipf_router_bias whose realised routing of tokens ``x`` (float64 router on the
    RMS-normed rows, bf16 bias) is closest to the ideal Zipf(s) entry counts in log space.
    Returns (gamma, realised counts by rank)."""
    T, E, K = x.shape[0], layer.num_experts, layer.experts_per_token
    x64 = x.astype(np.float64)
    xn = x64 / np.sqrt((x64 * x64).mean(1, keepdims=True) + layer.rms_eps)
    if layer.gamma_f32 is not None:
        xn = xn * layer.gamma_f32.astype(np.float64)
    base = xn @ layer.router_w_f32.astype(np.float64).T
    ideal = np.log(zipf_ideal_counts(E, s, T, K))
    best = None
    for g in grid:
        b = round_bf16(zipf_router_bias(E, s, gamma=float(g), seed=seed)).astype(np.float64)
        c = zipf_rank_counts(base + b, K, E, seed)
        err = float(np.sum((np.log(np.maximum(c, 0.5)) - ideal) ** 2))
        if best is None or err < best[0]:
            best = (err, round(float(g), 2), c)
    return best[1], best[2]


# Benchmark configurations (D, F, E, k, T, activation dtype).
CONFIGS = {
    "tiny": dict(d_model=256, ffn_hidden=256, num_experts=2, experts_per_token=2, tokens=16, dtype="f32"),
    "20b_decode": dict(d_model=2880, ffn_hidden=2880, num_experts=32, experts_per_token=4, tokens=8, dtype="bf16"),
    "20b_prefill": dict(d_model=2880, ffn_hidden=2880, num_experts=32, experts_per_token=4, tokens=4096,
                        dtype="bf16"),
    "120b": dict(d_model=2880, ffn_hidden=2880, num_experts=128, experts_per_token=4, tokens=64, dtype="bf16"),
}


def decode_bytes(layer: MoeLayerData, touched: int, n_tokens: int, act_bytes: int) -> int:
    """Algorithmic HBM bytes of one layer forward: every touched expert's weights once, the
    router weight and bias, activations in and out."""
    E, D = layer.num_experts, layer.d_model
    sw = 2 if layer.dtype == "bf16" else 4
    return touched * layer.expert_bytes() + E * D * sw + E * sw + 2 * n_tokens * D * act_bytes


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)


__all__ = ["MoeLayerData", "make_layer", "make_tokens", "zipf_router_bias", "ZIPF_GAMMA_C3", "calibrate_zipf_gamma",
           "zipf_rank_counts", "zipf_rank_counts_from_idx", "zipf_ideal_counts", "f32_to_bf16_bits", "bf16_bits_to_f32",
           "round_bf16", "CONFIGS", "decode_bytes", "ceil_div", "math"]
