"""On-disk MoE weights -> ``MoeLayerData`` for ``MoeLayer`` (the resident upload).

Two formats, as the reference reads them:

* **model.bin** (``GPT-OSS v1.0``): a sequential file -- header, tokenizer, 16 KiB alignment,
  embedding, per-layer attention / norm / router tensors (16-byte aligned), final norm and
  unembedding, then per layer (16 KiB aligned) and per expert (each 16-byte aligned): W1 blocks,
  W1 scales (+14 mod 256), b1 (bf16), W2 blocks, W2 scales (+14), b2 (bf16).  Reader: reference
  ``src/loader/modelbin.rs:77-458``; MoE writer: ``src/bin/gptoss_export.rs:528-593``.  The MoE
  layer takes the scales as stored with ``ue8_offset = 14`` (``src/loader/modelbin.rs:452-453``),
  the router (``mlp.gate``) and RmsNorm scale (``mlp.norm``) from the per-layer section.
* **safetensors** (original GPT-OSS checkpoint naming, ``block.{l}.mlp.mlp1_weight.blocks`` etc.,
  blocks ``[E, rows, G, 16]`` u8, scales ``[E, rows, G]`` u8 raw e8m0, biases / router / norm
  bf16): reference ``src/loader/gpt_oss.rs:350-423`` and ``src/loader/mxfp4.rs:81-125``.

W1 row order: the reference's resident kernel pairs gate row ``f`` with linear row ``F + f``
(``src/quant/gpu.rs:112-113``) -- the model.bin path; its dense safetensors path dequantises W1
into a Linear consumed by the interleaved SwiGLU (``src/activation/mod.rs:5-45``).  The loaders
default to those two (``halves`` for model.bin, ``interleaved`` for safetensors); pass
``gate_up_layout`` to choose.

Nothing here touches the GPU: the arrays are memory-mapped and copied once into the
``MoeLayerData`` host buffers, which ``MoeLayer`` uploads.
"""
from __future__ import annotations

import dataclasses
import json
import struct

import numpy as np

from .synth import MoeLayerData, bf16_bits_to_f32, f32_to_bf16_bits

MODELBIN_MAGIC = b"GPT-OSS v1.0"
SWIGLU_ALPHA = 1.702  # hard-coded by the reference kernel (src/quant/gpu.rs:144)


def _align(off: int, a: int) -> int:
    return off if off % a == 0 else off + (a - off % a)


# ---------------------------------------------------------------------------------------------
# model.bin
# ---------------------------------------------------------------------------------------------
@dataclasses.dataclass
class ModelBinHeader:
    """Fields of the model.bin header and tokenizer header (reference src/loader/modelbin.rs:45-66,
    parse order :77-125)."""

    context_length: int
    num_blocks: int
    num_experts: int
    num_active_experts: int
    embedding_dim: int
    mlp_dim: int
    swiglu_limit: float
    head_dim: int
    num_heads: int
    num_kv_heads: int
    attention_window: int
    rope_theta: float
    interpolation_scale: float
    yarn_offset: float
    yarn_scale: float
    yarn_multiplier: float
    rms_eps: float
    num_special: int = 0
    num_text: int = 0
    regex_size: int = 0
    tokens_size: int = 0
    after_tokenizer: int = 0  # file offset of the embedding (16 KiB aligned)

    @property
    def included_tokens(self) -> int:
        return self.num_text + self.num_special


_HDR_FMT = "<6If4I6f"  # context_length .. mlp_dim, swiglu_limit, head_dim .. window, rope .. rms_eps


def read_modelbin_header(path) -> ModelBinHeader:
    with open(path, "rb") as f:
        magic = f.read(16)
        if magic[:12] != MODELBIN_MAGIC:
            raise ValueError(f"{path}: invalid magic header (expected {MODELBIN_MAGIC!r})")
        f.read(16)  # model uuid
        vals = struct.unpack(_HDR_FMT, f.read(struct.calcsize(_HDR_FMT)))
        f.read(16)  # layout uuid
        f.read(16)  # tokenizer uuid
        num_special, num_text, regex_size, tokens_size = struct.unpack("<4I", f.read(16))
        off = f.tell() + num_special * 16 + regex_size + tokens_size
    h = ModelBinHeader(*vals)
    h.num_special, h.num_text, h.regex_size, h.tokens_size = num_special, num_text, regex_size, tokens_size
    h.after_tokenizer = _align(off, 16384)
    return h


@dataclasses.dataclass
class _ModelBinLayout:
    """File offsets of what the MoE layer needs (computed by walking the reference's order)."""

    norm: list      # per layer: offset of mlp.norm.scale [D] bf16
    gate: list      # per layer: offset of mlp.gate.weight [E, D] bf16 (bias [E] follows)
    experts: list   # per layer, per expert: (w1b, w1s, b1, w2b, w2s, b2) offsets
    end: int


def _modelbin_layout(h: ModelBinHeader) -> _ModelBinLayout:
    D, F, E, L = h.embedding_dim, h.mlp_dim, h.num_experts, h.num_blocks
    qkv_rows = h.head_dim * (h.num_heads + 2 * h.num_kv_heads)
    off = h.after_tokenizer + h.included_tokens * D * 2  # embedding (src/loader/modelbin.rs:178-185)
    norm, gate = [], []
    for _ in range(L):  # :187-296
        off = _align(off, 16) + D * 2                                # norm_attn
        off = _align(off, 16) + qkv_rows * D * 2 + qkv_rows * 2      # qkv weight + bias
        off = _align(off, 16) + h.num_heads * 2                      # sinks
        off = _align(off, 16) + D * h.num_heads * h.head_dim * 2 + D * 2  # attn out weight + bias
        off = _align(off, 16)
        norm.append(off)
        off += D * 2                                                 # mlp.norm.scale
        off = _align(off, 16)
        gate.append(off)
        off += E * D * 2 + E * 2                                     # mlp.gate weight + bias
    off = _align(off, 16) + D * 2                                    # norm_final (:297-300)
    off = _align(off, 16) + h.included_tokens * D * 2                # unembedding (:302-308)
    r1, r2 = 2 * F, D
    bpr1, bpr2, gpr1, gpr2 = (D + 1) // 2, (F + 1) // 2, (D + 31) // 32, (F + 31) // 32
    experts = []
    for _ in range(L):  # :338-405
        off = _align(off, 16384)
        per = []
        for _ in range(E):
            w1b = _align(off, 16); off = w1b + r1 * bpr1
            w1s = _align(off, 16); off = w1s + r1 * gpr1
            b1 = _align(off, 16); off = b1 + r1 * 2
            w2b = _align(off, 16); off = w2b + r2 * bpr2
            w2s = _align(off, 16); off = w2s + r2 * gpr2
            b2 = _align(off, 16); off = b2 + r2 * 2
            per.append((w1b, w1s, b1, w2b, w2s, b2))
        experts.append(per)
    return _ModelBinLayout(norm, gate, experts, off)


GATE_UP_LAYOUTS = ("interleaved", "halves")


def load_modelbin_moe(path, layers=None, gate_up_layout: str = "interleaved") -> list[MoeLayerData]:
    """The MoE layers of a model.bin as ``MoeLayerData`` (bf16 biases / router / norm, scales as
    stored with ``ue8_offset`` 14).  ``layers``: indices to load (default all).

    ``gate_up_layout`` names the row order of the stored mlp1 (W1) rows and b1:
      * "interleaved" (default): row 2f is the gate and row 2f + 1 the linear unit of feature f.
        The exporter copies GPT-OSS checkpoint rows verbatim (src/bin/gptoss_export.rs:553-555)
        and the checkpoints interleave them (the crate's own swiglu_clamp pairs them so,
        src/activation/mod.rs:5-12), so this is the layer a real model.bin holds.
      * "halves": rows [0, F) gate and [F, 2F) linear -- the pairing the reference's resident
        kernel applies to whatever it is given (src/quant/gpu.rs:112-113, src/moe/mod.rs:336-337).
        Opt in to reproduce that kernel's outputs on a real file bit for bit in row pairing."""
    if gate_up_layout not in GATE_UP_LAYOUTS:
        raise ValueError(f"gate_up_layout must be one of {GATE_UP_LAYOUTS}, got {gate_up_layout!r}")
    h = read_modelbin_header(path)
    lay = _modelbin_layout(h)
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    if mm.shape[0] < lay.end:
        raise ValueError(f"{path}: truncated ({mm.shape[0]} bytes, the MoE sections end at {lay.end})")
    D, F, E = h.embedding_dim, h.mlp_dim, h.num_experts
    r1, r2 = 2 * F, D
    bpr1, bpr2, gpr1, gpr2 = (D + 1) // 2, (F + 1) // 2, (D + 31) // 32, (F + 31) // 32

    def bf16(off, n):
        return bf16_bits_to_f32(np.frombuffer(mm, dtype=np.uint16, count=n, offset=off))

    out = []
    for l in range(h.num_blocks) if layers is None else layers:
        ex = lay.experts[l]
        w1b = np.empty((E, r1, bpr1), np.uint8)
        w1s = np.empty((E, r1, gpr1), np.uint8)
        w2b = np.empty((E, r2, bpr2), np.uint8)
        w2s = np.empty((E, r2, gpr2), np.uint8)
        b1 = np.empty((E, r1), np.float32)
        b2 = np.empty((E, r2), np.float32)
        for e, (o1b, o1s, ob1, o2b, o2s, ob2) in enumerate(ex):
            w1b[e] = mm[o1b:o1b + r1 * bpr1].reshape(r1, bpr1)
            w1s[e] = mm[o1s:o1s + r1 * gpr1].reshape(r1, gpr1)
            b1[e] = bf16(ob1, r1)
            w2b[e] = mm[o2b:o2b + r2 * bpr2].reshape(r2, bpr2)
            w2s[e] = mm[o2s:o2s + r2 * gpr2].reshape(r2, gpr2)
            b2[e] = bf16(ob2, r2)
        out.append(MoeLayerData(
            d_model=D, ffn_hidden=F, num_experts=E, experts_per_token=h.num_active_experts,
            w1_blocks=w1b, w1_scales=w1s, w2_blocks=w2b, w2_scales=w2s, b1_f32=b1, b2_f32=b2,
            router_w_f32=bf16(lay.gate[l], E * D).reshape(E, D), router_b_f32=bf16(lay.gate[l] + E * D * 2, E),
            dtype="bf16", ue8_offset=14, gate_up_layout=gate_up_layout, swiglu_alpha=SWIGLU_ALPHA,
            swiglu_limit=float(h.swiglu_limit), rms_eps=float(h.rms_eps), gamma_f32=bf16(lay.norm[l], D)))
    return out


def write_modelbin(path, h: ModelBinHeader, layers: list[MoeLayerData], fill_seed: int | None = None) -> None:
    """Writes a model.bin in the reference's order (for round trips and synthetic files).  The MoE
    sections, the per-layer router and RmsNorm scale come from ``layers`` (scale bytes written as
    stored in the layer plus 14 - its ``ue8_offset``, mod 256, the exporter's wrapping add); every
    other tensor is zeros, or seeded bytes with ``fill_seed``.  Tokenizer blobs are zeros."""
    D, F, E, L = h.embedding_dim, h.mlp_dim, h.num_experts, h.num_blocks
    assert len(layers) == L
    for d in layers:
        assert (d.d_model, d.ffn_hidden, d.num_experts) == (D, F, E)
    rng = np.random.default_rng(fill_seed) if fill_seed is not None else None

    def filler(n):
        return bytes(n) if rng is None else rng.integers(0, 256, n, dtype=np.uint8).tobytes()

    def bf16b(a):
        return f32_to_bf16_bits(np.asarray(a, np.float32)).tobytes()

    with open(path, "wb") as f:
        def pad(a):
            f.write(bytes(_align(f.tell(), a) - f.tell()))

        f.write(MODELBIN_MAGIC + bytes(4))
        f.write(bytes(16))
        f.write(struct.pack(_HDR_FMT, h.context_length, L, E, h.num_active_experts, D, F, h.swiglu_limit,
                            h.head_dim, h.num_heads, h.num_kv_heads, h.attention_window, h.rope_theta,
                            h.interpolation_scale, h.yarn_offset, h.yarn_scale, h.yarn_multiplier, h.rms_eps))
        f.write(bytes(16))
        f.write(bytes(16))
        f.write(struct.pack("<4I", h.num_special, h.num_text, h.regex_size, h.tokens_size))
        f.write(bytes(h.num_special * 16 + h.regex_size + h.tokens_size))
        pad(16384)
        f.write(filler(h.included_tokens * D * 2))
        qkv = h.head_dim * (h.num_heads + 2 * h.num_kv_heads)
        for d in layers:
            pad(16); f.write(filler(D * 2))
            pad(16); f.write(filler(qkv * D * 2 + qkv * 2))
            pad(16); f.write(filler(h.num_heads * 2))
            pad(16); f.write(filler(D * h.num_heads * h.head_dim * 2 + D * 2))
            pad(16); f.write(bf16b(d.gamma_f32 if d.gamma_f32 is not None else np.ones(D, np.float32)))
            pad(16); f.write(bf16b(d.router_w_f32)); f.write(bf16b(d.router_b_f32))
        pad(16); f.write(filler(D * 2))
        pad(16); f.write(filler(h.included_tokens * D * 2))
        for d in layers:
            pad(16384)
            off = (14 - d.ue8_offset) % 256
            for e in range(E):
                pad(16); f.write(np.ascontiguousarray(d.w1_blocks[e], np.uint8).tobytes())
                pad(16); f.write(((np.asarray(d.w1_scales[e], np.int32) + off) % 256).astype(np.uint8).tobytes())
                pad(16); f.write(bf16b(d.b1_f32[e]))
                pad(16); f.write(np.ascontiguousarray(d.w2_blocks[e], np.uint8).tobytes())
                pad(16); f.write(((np.asarray(d.w2_scales[e], np.int32) + off) % 256).astype(np.uint8).tobytes())
                pad(16); f.write(bf16b(d.b2_f32[e]))


# ---------------------------------------------------------------------------------------------
# safetensors (original GPT-OSS checkpoint naming)
# ---------------------------------------------------------------------------------------------
_ST_DTYPES = {"U8": np.uint8, "BF16": np.uint16, "F32": np.float32, "F16": np.float16, "I32": np.int32}


def read_safetensors(path) -> dict:
    """name -> (dtype string, numpy view over the memory-mapped file).  BF16 tensors are uint16
    bit patterns.  Format: u64 LE header length, JSON header, raw little-endian data."""
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    n = int(np.frombuffer(mm, dtype="<u8", count=1)[0])
    hdr = json.loads(bytes(mm[8:8 + n]).decode("utf-8"))
    base = 8 + n
    out = {}
    for name, meta in hdr.items():
        if name == "__metadata__":
            continue
        dt = _ST_DTYPES.get(meta["dtype"])
        if dt is None:
            raise ValueError(f"{path}: tensor {name}: unsupported dtype {meta['dtype']}")
        s, e = meta["data_offsets"]
        shape = tuple(meta["shape"])
        arr = np.frombuffer(mm, dtype=dt, count=(e - s) // np.dtype(dt).itemsize, offset=base + s)
        out[name] = (meta["dtype"], arr.reshape(shape))
    return out


def write_safetensors(path, tensors: dict) -> None:
    """tensors: name -> (dtype string, numpy array of the matching storage type)."""
    hdr, blobs, off = {}, [], 0
    for name, (dt, arr) in tensors.items():
        b = np.ascontiguousarray(arr, dtype=_ST_DTYPES[dt]).tobytes()
        hdr[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(hdr).encode("utf-8")
    h += b" " * (_align(len(h), 8) - len(h))
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def gptoss_moe_tensor_names(l: int) -> dict:
    """The checkpoint names the reference maps for layer l (src/loader/gpt_oss.rs:350-423)."""
    p = f"block.{l}.mlp."
    return {"w1b": p + "mlp1_weight.blocks", "w1s": p + "mlp1_weight.scales", "b1": p + "mlp1_bias",
            "w2b": p + "mlp2_weight.blocks", "w2s": p + "mlp2_weight.scales", "b2": p + "mlp2_bias",
            "gw": p + "gate.weight", "gb": p + "gate.bias", "norm": p + "norm.scale"}


def load_safetensors_moe(path, layer: int, experts_per_token: int = 4, gate_up_layout: str = "interleaved",
                         swiglu_limit: float = 7.0, rms_eps: float = 1e-5) -> MoeLayerData:
    """MoE layer ``layer`` of an original GPT-OSS safetensors checkpoint (scales raw e8m0,
    ``ue8_offset`` 0).  The checkpoint carries no config: top-k, SwiGLU limit and RmsNorm epsilon
    are arguments (GPT-OSS values by default)."""
    st = read_safetensors(path)
    nm = gptoss_moe_tensor_names(layer)
    missing = [v for v in nm.values() if v not in st]
    if missing:
        raise KeyError(f"{path}: missing tensors {missing}")

    def u8(k):
        dt, a = st[nm[k]]
        if dt != "U8":
            raise ValueError(f"{nm[k]}: expected U8, got {dt}")
        return a

    def fl(k):
        dt, a = st[nm[k]]
        return bf16_bits_to_f32(a) if dt == "BF16" else np.asarray(a, np.float32)

    w1b, w1s, w2b, w2s = u8("w1b"), u8("w1s"), u8("w2b"), u8("w2s")
    E, r1 = w1b.shape[0], w1b.shape[1]
    D = w2b.shape[1]
    F = r1 // 2
    if w1b.ndim != 4 or w1b.shape[3] != 16 or w1s.shape != w1b.shape[:3] or w2s.shape != w2b.shape[:3]:
        raise ValueError(f"{path}: MXFP4 tensors of layer {layer} are not [E, rows, G, 16] + [E, rows, G]")
    dtype = "bf16" if st[nm["b1"]][0] == "BF16" else "f32"
    return MoeLayerData(
        d_model=D, ffn_hidden=F, num_experts=E, experts_per_token=experts_per_token,
        w1_blocks=np.ascontiguousarray(w1b.reshape(E, r1, -1)), w1_scales=np.ascontiguousarray(w1s),
        w2_blocks=np.ascontiguousarray(w2b.reshape(E, D, -1)), w2_scales=np.ascontiguousarray(w2s),
        b1_f32=fl("b1").reshape(E, r1).copy(), b2_f32=fl("b2").reshape(E, D).copy(),
        router_w_f32=fl("gw").reshape(E, D).copy(), router_b_f32=fl("gb").reshape(E).copy(),
        dtype=dtype, ue8_offset=0, gate_up_layout=gate_up_layout, swiglu_alpha=SWIGLU_ALPHA,
        swiglu_limit=swiglu_limit, rms_eps=rms_eps, gamma_f32=fl("norm").reshape(D).copy())
