"""Python host front-end over the C ABI, mirroring the reference's MoE module surface.

Reference surface (ariawisp/burn-extended):
  MoeConfig {d_model, ffn_hidden, num_experts, experts_per_token, swiglu_alpha, swiglu_limit, disabled}
                                              src/moe/mod.rs:22-33
  MoeGatedSwiGLU::set_resident(resident)      src/moe/mod.rs:95-97
  MoeGatedSwiGLU::forward(x) -> x + MoE(RmsNorm(x))   src/moe/mod.rs:99-115 (panics without resident)
  QuantLinearMxFp4Desc / MoeQuantLayerHost    src/quant/mod.rs:3-21
  MoeQuantLayerResident::new(device, ...)     src/quant/gpu.rs:30-54

Device tensors are torch tensors (HIP memory); kernels run on the current torch stream.
"""
from __future__ import annotations

import ctypes
import dataclasses

import numpy as np
import torch

from . import _native as N
from .synth import MoeLayerData, f32_to_bf16_bits


@dataclasses.dataclass
class QuantLinearMxFp4Desc:
    """Mirror of QuantLinearMxFp4Desc (src/quant/mod.rs:3-11)."""
    experts: int
    rows: int
    cols: int
    bpr: int
    gpr: int
    ue8_offset: int = 0

    @classmethod
    def for_matrix(cls, experts, rows, cols, ue8_offset=0):
        return cls(experts, rows, cols, (cols + 1) // 2, (cols + 31) // 32, ue8_offset)

    def c(self) -> N.MxFp4Desc:
        return N.MxFp4Desc(self.experts, self.rows, self.cols, self.bpr, self.gpr, self.ue8_offset)


@dataclasses.dataclass
class MoeQuantLayerHost:
    """Mirror of MoeQuantLayerHost (src/quant/mod.rs:13-21): flat expert-major u8 payloads."""
    w1_desc: QuantLinearMxFp4Desc
    w2_desc: QuantLinearMxFp4Desc
    w1_blocks: np.ndarray
    w1_scales: np.ndarray
    w2_blocks: np.ndarray
    w2_scales: np.ndarray


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _x_dtype(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return N.BURNEXT_BF16
    if t.dtype == torch.float32:
        return N.BURNEXT_F32
    raise TypeError(f"activations must be bfloat16 or float32, got {t.dtype}")


def _stream(stream) -> ctypes.c_void_p:
    s = torch.cuda.current_stream() if stream is None else stream
    return ctypes.c_void_p(s.cuda_stream)


class MoeLayer:
    """One device-resident MoE layer (burnext_moe_layer_create / _destroy)."""

    def __init__(self, data: MoeLayerData, device: int = 0, gate_up_layout: str | None = None, disabled: bool = False):
        self.data = data
        self.device = device
        D, F, E, K = data.d_model, data.ffn_hidden, data.num_experts, data.experts_per_token
        self.k = min(max(K, 1), E)
        cfg = N.MoeConfigC(D, F, E, K, data.swiglu_alpha, data.swiglu_limit, data.rms_eps,
                           1 if disabled else 0)
        d1 = N.MxFp4Desc.for_matrix(E, 2 * F, D, data.ue8_offset)
        d2 = N.MxFp4Desc.for_matrix(E, D, F, data.ue8_offset)
        arrs = {k: np.ascontiguousarray(getattr(data, k)) for k in ("w1_blocks", "w1_scales", "w2_blocks", "w2_scales")}
        if data.dtype == "bf16":
            dt = N.BURNEXT_BF16
            b1, b2 = data.b1_bits, data.b2_bits
            rw, rb = data.router_w_bits, data.router_b_bits
            g = None if data.gamma_f32 is None else f32_to_bf16_bits(data.gamma_f32)
        else:
            dt = N.BURNEXT_F32
            b1, b2 = np.ascontiguousarray(data.b1_f32), np.ascontiguousarray(data.b2_f32)
            rw, rb = np.ascontiguousarray(data.router_w_f32), np.ascontiguousarray(data.router_b_f32)
            g = None if data.gamma_f32 is None else np.ascontiguousarray(data.gamma_f32)
        layout = {"halves": N.GATE_UP_HALVES, "interleaved": N.GATE_UP_INTERLEAVED}[gate_up_layout or
                                                                                     data.gate_up_layout]
        h = ctypes.c_void_p()
        N.check(N.lib().burnext_moe_layer_create(
            ctypes.byref(cfg), ctypes.byref(d1), _ptr(arrs["w1_blocks"]), _ptr(arrs["w1_scales"]), ctypes.byref(d2),
            _ptr(arrs["w2_blocks"]), _ptr(arrs["w2_scales"]), _ptr(b1), _ptr(b2), dt, _ptr(rw), _ptr(rb), dt,
            _ptr(g), dt, layout, device, ctypes.byref(h)))
        self.handle = h
        self._ws = {}  # stream handle -> (buffer, bytes, alignment offset)

    def close(self) -> None:
        if getattr(self, "handle", None) is not None and self.handle.value:
            N.lib().burnext_moe_layer_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def workspace_size(self, n_tokens: int) -> int:
        b = ctypes.c_uint64()
        N.check(N.lib().burnext_moe_workspace_size(self.handle, n_tokens, ctypes.byref(b)))
        return b.value

    def workspace(self, n_tokens: int, stream=None) -> torch.Tensor:
        """A 256-byte-aligned device workspace for n_tokens, cached per stream and grown on demand.

        Calls on one stream reuse it in stream order; another stream gets its own buffer (allocated
        on that stream), since forwards that run concurrently must not share a workspace."""
        s = torch.cuda.current_stream(self.device) if stream is None else stream
        need = self.workspace_size(n_tokens)
        cur = self._ws.get(s.cuda_stream)
        if cur is None or cur[1] < need:
            with torch.cuda.stream(s):
                raw = torch.empty(need + 256, dtype=torch.uint8, device=f"cuda:{self.device}")
            cur = (raw, need, (-raw.data_ptr()) % 256)
            self._ws[s.cuda_stream] = cur
        raw, _, off = cur
        return raw[off:off + need]

    def forward(self, x: torch.Tensor, flags: int = N.FORWARD_DEFAULT, out: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        assert x.is_cuda and x.is_contiguous() and x.shape[-1] == self.data.d_model
        n = x.numel() // self.data.d_model
        y = torch.empty_like(x) if out is None else out
        ws = self.workspace(n, stream) if workspace is None else workspace
        N.check(N.lib().burnext_moe_forward(self.handle, ctypes.c_void_p(x.data_ptr()), _x_dtype(x),
                                            ctypes.c_void_p(y.data_ptr()), n, flags,
                                            ctypes.c_void_p(ws.data_ptr()), ws.numel(), _stream(stream)))
        return y

    def forward_noalloc(self, x: torch.Tensor, out: torch.Tensor, flags: int = N.FORWARD_DEFAULT,
                        stream=None) -> torch.Tensor:
        """burnext_moe_forward_noalloc: the forward on the library's fixed per-GPU scratch (no
        workspace, nothing allocated here or in the library; `out` is the caller's)."""
        assert x.is_cuda and x.is_contiguous() and x.shape[-1] == self.data.d_model
        n = x.numel() // self.data.d_model
        N.check(N.lib().burnext_moe_forward_noalloc(self.handle, ctypes.c_void_p(x.data_ptr()), _x_dtype(x),
                                                    ctypes.c_void_p(out.data_ptr()), n, flags, _stream(stream)))
        return out

    def route(self, x: torch.Tensor, flags: int = N.APPLY_RMSNORM, stream=None):
        n = x.numel() // self.data.d_model
        idx = torch.empty((n, self.k), dtype=torch.int32, device=x.device)
        w = torch.empty((n, self.k), dtype=torch.float32, device=x.device)
        lg = torch.empty((n, self.data.num_experts), dtype=torch.float32, device=x.device)
        ws = self.workspace(n, stream)
        N.check(N.lib().burnext_moe_route(self.handle, ctypes.c_void_p(x.data_ptr()), _x_dtype(x), n, flags,
                                          ctypes.c_void_p(idx.data_ptr()), ctypes.c_void_p(w.data_ptr()),
                                          ctypes.c_void_p(lg.data_ptr()), ctypes.c_void_p(ws.data_ptr()),
                                          ws.numel(), _stream(stream)))
        return idx, w, lg

    def dispatch(self, topk_idx: torch.Tensor, stream=None):
        n = topk_idx.shape[0]
        seg = torch.empty(self.data.num_experts + 1, dtype=torch.int32, device=topk_idx.device)
        perm = torch.empty(n * self.k, dtype=torch.int32, device=topk_idx.device)
        ws = self.workspace(n, stream)
        N.check(N.lib().burnext_moe_dispatch(self.handle, ctypes.c_void_p(topk_idx.data_ptr()), n,
                                             ctypes.c_void_p(seg.data_ptr()), ctypes.c_void_p(perm.data_ptr()),
                                             ctypes.c_void_p(ws.data_ptr()), ws.numel(), _stream(stream)))
        return seg, perm

    def route_dispatch(self, x: torch.Tensor, flags: int = N.APPLY_RMSNORM, stream=None):
        """Routing and dispatch as the forward runs them for this batch size (for n <= 16 the
        fused one-workgroup kernel): (topk_idx, topk_w, seg_offsets, perm)."""
        n = x.numel() // self.data.d_model
        idx = torch.empty((n, self.k), dtype=torch.int32, device=x.device)
        w = torch.empty((n, self.k), dtype=torch.float32, device=x.device)
        seg = torch.empty(self.data.num_experts + 1, dtype=torch.int32, device=x.device)
        perm = torch.empty(n * self.k, dtype=torch.int32, device=x.device)
        ws = self.workspace(n, stream)
        N.check(N.lib().burnext_moe_route_dispatch(
            self.handle, ctypes.c_void_p(x.data_ptr()), _x_dtype(x), n, flags, ctypes.c_void_p(idx.data_ptr()),
            ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(seg.data_ptr()), ctypes.c_void_p(perm.data_ptr()),
            ctypes.c_void_p(ws.data_ptr()), ws.numel(), _stream(stream)))
        return idx, w, seg, perm

    def profile_enable(self, on: bool = True) -> None:
        N.check(N.lib().burnext_moe_profile_enable(self.handle, 1 if on else 0))

    def profile_read(self) -> dict:
        ms = (ctypes.c_double * N.NUM_KERNELS)()
        cnt = (ctypes.c_uint64 * N.NUM_KERNELS)()
        N.check(N.lib().burnext_moe_profile_read(self.handle, ms, cnt, N.NUM_KERNELS))
        return {N.KERNEL_NAMES[i]: (ms[i], cnt[i]) for i in range(N.NUM_KERNELS)}


def mxfp4_dequant(desc: QuantLinearMxFp4Desc, blocks: torch.Tensor, scales: torch.Tensor,
                  out_dtype=torch.float32, stream=None) -> torch.Tensor:
    """burnext_mxfp4_dequant on device tensors; returns [experts*rows, cols]."""
    out = torch.empty((desc.experts * desc.rows, desc.cols), dtype=out_dtype, device=blocks.device)
    dt = N.BURNEXT_BF16 if out_dtype == torch.bfloat16 else N.BURNEXT_F32
    cd = desc.c()
    N.check(N.lib().burnext_mxfp4_dequant(ctypes.byref(cd), ctypes.c_void_p(blocks.data_ptr()),
                                          ctypes.c_void_p(scales.data_ptr()), ctypes.c_void_p(out.data_ptr()), dt,
                                          _stream(stream)))
    return out


def to_device_x(x: np.ndarray, dtype: str, device: int = 0) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(x, np.float32))
    t = t.to(torch.bfloat16) if dtype == "bf16" else t
    return t.to(f"cuda:{device}")
