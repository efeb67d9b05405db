"""C-ABI checks that need no GPU: the library loads, exports exactly what include/burnext_moe.h
declares, and rejects bad arguments with the documented status and a message (the reference
panics or asserts on the same inputs, src/moe/mod.rs:111-113, src/quant/gpu.rs:30-54)."""
from __future__ import annotations

import ctypes
import pathlib
import re
import subprocess
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "burn-extended_amd"))

from burnext_amd import _native as N  # noqa: E402

HEADER = ROOT / "include" / "burnext_moe.h"
HEADERS = [HEADER, ROOT / "include" / "burnext_gptoss.h"]


def header_functions() -> list[str]:
    text = "".join(re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S) for h in HEADERS)
    return sorted(set(re.findall(r"\b(burnext_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    if not N.LIB_PATH.exists():
        pytest.skip("libburnext_moe.so not built (run __graft_entry__.build())")
    return N.lib()


def test_header_declares_the_binding_exports():
    assert header_functions() == sorted(N.EXPORTS)


def test_library_exports_every_declared_symbol(L):
    for name in header_functions():
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(N.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    missing = set(header_functions()) - exported
    assert not missing, missing
    # nothing else with the public prefix leaks out
    assert {s for s in exported if s.startswith("burnext_")} == set(header_functions())


def test_header_compiles_as_c():
    src = '#include "burnext_moe.h"\nint main(void){return (int)sizeof(burnext_mxfp4_desc);}\n'
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-I", str(HEADER.parent), "-x", "c",
                        "-"], input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_struct_layouts_match_header(L):
    # offsets of the mirrored structs as the C compiler lays them out
    src = r'''
#include <stddef.h>
#include <stdio.h>
#include "burnext_moe.h"
int main(void) {
  printf("%zu %zu %zu\n", sizeof(burnext_mxfp4_desc), offsetof(burnext_mxfp4_desc, ue8_offset),
         sizeof(burnext_moe_config));
  printf("%zu %zu\n", offsetof(burnext_moe_config, swiglu_alpha), offsetof(burnext_moe_config, disabled));
  return 0;
}
'''
    exe = ROOT / "oracle" / "_build" / "abi_layout"
    exe.parent.mkdir(parents=True, exist_ok=True)
    r = subprocess.run(["gcc", "-std=c99", "-I", str(HEADER.parent), "-x", "c", "-", "-o", str(exe)], input=src,
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    vals = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert vals[0] == ctypes.sizeof(N.MxFp4Desc)
    assert vals[1] == N.MxFp4Desc.ue8_offset.offset
    assert vals[2] == ctypes.sizeof(N.MoeConfigC)
    assert vals[3] == N.MoeConfigC.swiglu_alpha.offset
    assert vals[4] == N.MoeConfigC.disabled.offset


def _cfg(D=64, F=64, E=4, K=2):
    return N.MoeConfigC(D, F, E, K, 1.702, 7.0, 1e-5, 0)


def _create(L, cfg, w1d, w2d, bias_dtype=N.BURNEXT_F32, router_dtype=N.BURNEXT_F32, layout=N.GATE_UP_INTERLEAVED,
            null=()):
    D, F, E = cfg.d_model, cfg.ffn_hidden, cfg.num_experts
    bufs = {
        "w1b": np.zeros(max(1, E * 2 * F * ((D + 1) // 2)), np.uint8),
        "w1s": np.zeros(max(1, E * 2 * F * ((D + 31) // 32)), np.uint8),
        "w2b": np.zeros(max(1, E * D * ((F + 1) // 2)), np.uint8),
        "w2s": np.zeros(max(1, E * D * ((F + 31) // 32)), np.uint8),
        "b1": np.zeros(max(1, E * 2 * F), np.float32),
        "b2": np.zeros(max(1, E * D), np.float32),
        "rw": np.zeros(max(1, E * D), np.float32),
    }
    p = {k: (None if k in null else v.ctypes.data_as(ctypes.c_void_p)) for k, v in bufs.items()}
    out = ctypes.c_void_p()
    st = L.burnext_moe_layer_create(ctypes.byref(cfg), ctypes.byref(w1d), p["w1b"], p["w1s"], ctypes.byref(w2d),
                                    p["w2b"], p["w2s"], p["b1"], p["b2"], bias_dtype, p["rw"], None, router_dtype,
                                    None, N.BURNEXT_F32, layout, 0, ctypes.byref(out))
    return st, out


def _descs(cfg):
    D, F, E = cfg.d_model, cfg.ffn_hidden, cfg.num_experts
    return N.MxFp4Desc.for_matrix(E, 2 * F, D), N.MxFp4Desc.for_matrix(E, D, F)


def test_create_rejects_null_out(L):
    cfg = _cfg()
    w1d, w2d = _descs(cfg)
    st = L.burnext_moe_layer_create(ctypes.byref(cfg), ctypes.byref(w1d), None, None, ctypes.byref(w2d), None, None,
                                    None, None, 0, None, None, 0, None, 0, 1, 0, None)
    assert st == N.BURNEXT_INVALID_ARG
    assert "out_layer" in N.last_error()


@pytest.mark.parametrize("which", ["w1b", "w1s", "w2b", "w2s", "b1", "b2", "rw"])
def test_create_rejects_null_buffers(L, which):
    cfg = _cfg()
    w1d, w2d = _descs(cfg)
    st, out = _create(L, cfg, w1d, w2d, null=(which,))
    assert st == N.BURNEXT_INVALID_ARG and not out.value
    assert "null" in N.last_error()


@pytest.mark.parametrize("field,value", [("rows", 63), ("cols", 65), ("bpr", 31), ("gpr", 3), ("experts", 5),
                                         ("ue8_offset", -1), ("ue8_offset", 256)])
def test_create_rejects_descriptor_mismatch(L, field, value):
    cfg = _cfg()
    w1d, w2d = _descs(cfg)
    setattr(w1d, field, value)
    st, out = _create(L, cfg, w1d, w2d)
    assert st == N.BURNEXT_INVALID_ARG and not out.value
    assert "w1 descriptor" in N.last_error()
    w1d, w2d = _descs(cfg)
    setattr(w2d, field, value)
    st, _ = _create(L, cfg, w1d, w2d)
    assert st == N.BURNEXT_INVALID_ARG
    assert "w2 descriptor" in N.last_error()


def test_create_rejects_bad_enums_and_shapes(L):
    cfg = _cfg()
    w1d, w2d = _descs(cfg)
    assert _create(L, cfg, w1d, w2d, bias_dtype=7)[0] == N.BURNEXT_INVALID_ARG
    assert _create(L, cfg, w1d, w2d, router_dtype=-1)[0] == N.BURNEXT_INVALID_ARG
    assert _create(L, cfg, w1d, w2d, layout=2)[0] == N.BURNEXT_INVALID_ARG
    assert "gate_up_layout" in N.last_error()
    z = _cfg(D=0)
    assert _create(L, z, *_descs(z))[0] == N.BURNEXT_INVALID_ARG
    big = _cfg(E=257)
    assert _create(L, big, *_descs(big))[0] == N.BURNEXT_UNSUPPORTED
    assert "256" in N.last_error()


def test_calls_on_null_layer(L):
    b = ctypes.c_uint64()
    assert L.burnext_moe_workspace_size(None, 8, ctypes.byref(b)) == N.BURNEXT_INVALID_ARG
    assert L.burnext_moe_forward(None, None, 0, None, 8, 3, None, 0, None) == N.BURNEXT_INVALID_ARG
    assert "layer is null" in N.last_error()
    assert L.burnext_moe_route(None, None, 0, 8, 1, None, None, None, None, 0, None) == N.BURNEXT_INVALID_ARG
    assert L.burnext_moe_dispatch(None, None, 8, None, None, None, 0, None) == N.BURNEXT_INVALID_ARG
    assert L.burnext_moe_profile_enable(None, 1) == N.BURNEXT_INVALID_ARG
    ms = (ctypes.c_double * N.NUM_KERNELS)()
    cnt = (ctypes.c_uint64 * N.NUM_KERNELS)()
    assert L.burnext_moe_profile_read(None, ms, cnt, N.NUM_KERNELS) == N.BURNEXT_INVALID_ARG
    L.burnext_moe_layer_destroy(None)  # no-op


def test_dequant_argument_checks(L):
    d = N.MxFp4Desc.for_matrix(1, 4, 64)
    buf = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    assert L.burnext_mxfp4_dequant(None, buf, buf, buf, 0, None) == N.BURNEXT_INVALID_ARG
    assert L.burnext_mxfp4_dequant(ctypes.byref(d), buf, buf, buf, 5, None) == N.BURNEXT_INVALID_ARG
    assert "out_dtype" in N.last_error()
    bad = N.MxFp4Desc(1, 4, 64, 31, 2, 0)
    assert L.burnext_mxfp4_dequant(ctypes.byref(bad), buf, buf, buf, 0, None) == N.BURNEXT_INVALID_ARG
    assert "bpr" in N.last_error()


def test_last_error_is_thread_local(L):
    import threading
    cfg = _cfg(E=257)
    _create(L, cfg, *_descs(cfg))
    seen = []
    t = threading.Thread(target=lambda: seen.append(N.last_error()))
    t.start()
    t.join()
    assert seen == [""]
    assert "256" in N.last_error()


# ---- include/burnext_gptoss.h -------------------------------------------------------------------

def test_gptoss_struct_layouts_match_header():
    src = r'''
#include <stddef.h>
#include <stdio.h>
#include "burnext_gptoss.h"
int main(void) {
  printf("%zu %zu %zu %zu %zu %zu %zu\n", sizeof(burnext_gptoss_config), offsetof(burnext_gptoss_config, kv_bf16),
         offsetof(burnext_gptoss_config, rms_eps), offsetof(burnext_gptoss_config, scale_dk),
         offsetof(burnext_gptoss_config, sink_tokens), offsetof(burnext_gptoss_config, experts_bf16),
         sizeof(burnext_gptoss_weights));
  printf("%zu %zu\n", offsetof(burnext_gptoss_weights, sinks), offsetof(burnext_gptoss_weights, lm_head));
  return 0;
}
'''
    exe = ROOT / "oracle" / "_build" / "abi_layout_gptoss"
    exe.parent.mkdir(parents=True, exist_ok=True)
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", str(HEADER.parent), "-x", "c", "-", "-o",
                        str(exe)], input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    vals = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert vals == [ctypes.sizeof(N.GptOssConfigC), N.GptOssConfigC.kv_bf16.offset, N.GptOssConfigC.rms_eps.offset,
                    N.GptOssConfigC.scale_dk.offset, N.GptOssConfigC.sink_tokens.offset,
                    N.GptOssConfigC.experts_bf16.offset, ctypes.sizeof(N.GptOssWeightsC), N.GptOssWeightsC.sinks.offset,
                    N.GptOssWeightsC.lm_head.offset]


def _gcfg(**kw):
    base = dict(vocab_size=64, d_model=64, n_layers=2, n_heads=4, kv_heads=2, head_dim=16, max_batch=4, cache_len=32,
                window_policy=2, window=8, full_on_even=1, rope_head_stride=1, max_positions=64, kv_bf16=0, rms_eps=1e-5,
                rope_theta=150000.0, rope_scaling_factor=32.0, rope_initial_context=4096.0, rope_ntk_alpha=1.0,
                rope_ntk_beta=32.0, scale_dk=1.0)
    base.update(kw)
    return N.GptOssConfigC(**base)


def _gweights():
    buf = np.zeros(1 << 16, np.uint16)
    p = buf.ctypes.data_as(ctypes.c_void_p)
    return N.GptOssWeightsC(*([p] * 13)), buf


@pytest.mark.parametrize("kw,status,msg", [
    (dict(head_dim=12), N.BURNEXT_UNSUPPORTED, "head_dim"),
    (dict(head_dim=136), N.BURNEXT_UNSUPPORTED, "head_dim"),
    (dict(n_heads=6, kv_heads=2), N.BURNEXT_UNSUPPORTED, "power of two"),
    (dict(n_heads=5, kv_heads=2), N.BURNEXT_UNSUPPORTED, "power of two"),
    (dict(n_heads=64, kv_heads=2), N.BURNEXT_UNSUPPORTED, "power of two"),
    (dict(max_batch=17), N.BURNEXT_UNSUPPORTED, "max_batch"),
    (dict(d_model=63), N.BURNEXT_UNSUPPORTED, "d_model"),
    (dict(vocab_size=0), N.BURNEXT_INVALID_ARG, "zero dimension"),
    (dict(cache_len=0), N.BURNEXT_INVALID_ARG, "zero dimension"),
    (dict(kv_bf16=2), N.BURNEXT_INVALID_ARG, "kv_bf16"),
    (dict(experts_bf16=2), N.BURNEXT_INVALID_ARG, "experts_bf16"),
    (dict(rope_head_stride=3), N.BURNEXT_INVALID_ARG, "rope_head_stride"),
    (dict(window=0), N.BURNEXT_INVALID_ARG, "window"),
    (dict(window_policy=3), N.BURNEXT_INVALID_ARG, "window_policy"),
    (dict(scale_dk=0.0), N.BURNEXT_INVALID_ARG, "scale_dk"),
    (dict(sink_tokens=32), N.BURNEXT_INVALID_ARG, "sink_tokens"),
    (dict(rope_theta=1.0), N.BURNEXT_INVALID_ARG, "rope_theta"),
    # YaRN thresholds: beta <= alpha makes low >= high (the reference asserts)
    (dict(rope_ntk_alpha=32.0, rope_ntk_beta=1.0), N.BURNEXT_INVALID_ARG, "YaRN"),
])
def test_gptoss_create_rejects_bad_config(L, kw, status, msg):
    cfg = _gcfg(**kw)
    w, _buf = _gweights()
    handles = (ctypes.c_void_p * 2)(1, 1)
    out = ctypes.c_void_p(123)
    st = L.burnext_gptoss_create(ctypes.byref(cfg), ctypes.byref(w), handles, 0, ctypes.byref(out))
    assert st == status, N.last_error()
    assert msg in N.last_error()
    assert not out.value


def test_gptoss_create_rejects_null_arguments(L):
    cfg = _gcfg()
    w, _buf = _gweights()
    handles = (ctypes.c_void_p * 2)(1, 1)
    out = ctypes.c_void_p()
    assert L.burnext_gptoss_create(ctypes.byref(cfg), ctypes.byref(w), handles, 0, None) == N.BURNEXT_INVALID_ARG
    assert L.burnext_gptoss_create(None, ctypes.byref(w), handles, 0, ctypes.byref(out)) == N.BURNEXT_INVALID_ARG
    assert L.burnext_gptoss_create(ctypes.byref(cfg), ctypes.byref(w), None, 0, ctypes.byref(out)) == \
        N.BURNEXT_INVALID_ARG
    w.wq = None
    assert L.burnext_gptoss_create(ctypes.byref(cfg), ctypes.byref(w), handles, 0, ctypes.byref(out)) == \
        N.BURNEXT_INVALID_ARG
    assert "weight" in N.last_error()
    w, _buf = _gweights()
    nulls = (ctypes.c_void_p * 2)(1, None)
    assert L.burnext_gptoss_create(ctypes.byref(cfg), ctypes.byref(w), nulls, 0, ctypes.byref(out)) == \
        N.BURNEXT_INVALID_ARG
    assert "MoE layer" in N.last_error()


def test_gptoss_calls_on_null_model(L):
    b = ctypes.c_uint64()
    assert L.burnext_gptoss_workspace_size(None, 1, ctypes.byref(b)) == N.BURNEXT_INVALID_ARG
    assert L.burnext_gptoss_reset(None) == N.BURNEXT_INVALID_ARG
    assert L.burnext_gptoss_cache_load(None, None, None, 1, 0, None) == N.BURNEXT_INVALID_ARG
    assert L.burnext_gptoss_decode(None, None, 1, 0, 0, None, None, None, None, 0, None) == N.BURNEXT_INVALID_ARG
    L.burnext_gptoss_destroy(None)  # no-op
