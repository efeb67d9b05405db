"""On-disk MoE weights: model.bin (reference src/loader/modelbin.rs:77-458, MoE writer
src/bin/gptoss_export.rs:528-593) and original-checkpoint safetensors (src/loader/gpt_oss.rs:350-423)
into MoeLayerData.  CPU round trips pin the byte layout; the GPU test runs a layer loaded from a
model.bin against the same layer built in memory and against the oracle."""
from __future__ import annotations

import dataclasses
import struct

import numpy as np
import pytest
import torch

from burnext_amd import loaders, synth

D, F, E, K = 64, 96, 4, 2


def _header(n_layers=2):
    return loaders.ModelBinHeader(
        context_length=4096, num_blocks=n_layers, num_experts=E, num_active_experts=K, embedding_dim=D, mlp_dim=F,
        swiglu_limit=7.0, head_dim=16, num_heads=4, num_kv_heads=2, attention_window=128, rope_theta=150000.0,
        interpolation_scale=32.0, yarn_offset=0.0, yarn_scale=1.0, yarn_multiplier=1.0, rms_eps=1e-5,
        num_special=3, num_text=10, regex_size=7, tokens_size=33)


def _layers(n=2, ue8=0):
    return [synth.make_layer(D, F, E, K, seed=11 + i, dtype="bf16", ue8_offset=ue8, with_gamma=True)
            for i in range(n)]


def _same_layer(a, b, scale_shift=0):
    for f in ("w1_blocks", "w2_blocks"):
        assert np.array_equal(getattr(a, f), getattr(b, f)), f
    for f in ("w1_scales", "w2_scales"):
        want = ((getattr(a, f).astype(np.int32) + scale_shift) % 256).astype(np.uint8)
        assert np.array_equal(want, getattr(b, f)), f
    for f in ("b1_f32", "b2_f32", "router_w_f32", "router_b_f32", "gamma_f32"):
        x, y = np.asarray(getattr(a, f), np.float32), np.asarray(getattr(b, f), np.float32)
        assert np.array_equal(x.reshape(-1).view(np.uint32), y.reshape(-1).view(np.uint32)), f


@pytest.mark.parametrize("ue8", [0, 14])
def test_modelbin_round_trip(tmp_path, ue8):
    src = _layers(ue8=ue8)
    path = tmp_path / "model.bin"
    loaders.write_modelbin(path, _header(), src, fill_seed=5)
    h = loaders.read_modelbin_header(path)
    assert (h.num_blocks, h.num_experts, h.num_active_experts, h.embedding_dim, h.mlp_dim) == (2, E, K, D, F)
    assert h.after_tokenizer % 16384 == 0
    got = loaders.load_modelbin_moe(path, gate_up_layout="interleaved")
    assert len(got) == 2
    for a, b in zip(src, got):
        assert b.ue8_offset == 14 and b.experts_per_token == K and b.gate_up_layout == "interleaved"
        assert b.swiglu_limit == 7.0 and abs(b.rms_eps - 1e-5) < 1e-12
        _same_layer(a, b, scale_shift=14 - ue8)  # stored = true + 14 (the exporter's wrapping add)
    # default: the checkpoints' interleaved rows; the reference kernel's halves pairing is opt-in
    assert loaders.load_modelbin_moe(path)[0].gate_up_layout == "interleaved"
    assert loaders.load_modelbin_moe(path, gate_up_layout="halves")[0].gate_up_layout == "halves"
    with pytest.raises(ValueError):
        loaders.load_modelbin_moe(path, gate_up_layout="split")


def test_modelbin_layout_alignment(tmp_path):
    """Byte positions the reference reader seeks to: 16 KiB before each MoE layer, 16 B before
    every expert tensor, and the first expert's W1 blocks start the first MoE layer exactly."""
    src = _layers()
    path = tmp_path / "model.bin"
    loaders.write_modelbin(path, _header(), src)
    h = loaders.read_modelbin_header(path)
    lay = loaders._modelbin_layout(h)
    raw = np.fromfile(path, dtype=np.uint8)
    assert raw.size == lay.end
    for l in range(2):
        first = lay.experts[l][0][0]
        assert first % 16384 == 0
        for ex in lay.experts[l]:
            assert all(o % 16 == 0 for o in ex)
        # W1 scales of expert 1 as stored: true exponent + 14
        o = lay.experts[l][1][1]
        assert np.array_equal(raw[o:o + 2 * F * (D // 32)], ((src[l].w1_scales[1].ravel().astype(int) + 14) % 256))
    # the header words the reference reads after the 16-byte magic and 16-byte uuid
    vals = struct.unpack("<6I", raw[32:56].tobytes())
    assert vals == (4096, 2, E, K, D, F)


def test_modelbin_rejects_bad_magic_and_truncation(tmp_path):
    path = tmp_path / "model.bin"
    loaders.write_modelbin(path, _header(1), _layers(1))
    data = bytearray(path.read_bytes())
    bad = tmp_path / "bad.bin"
    bad.write_bytes(b"NOT-GPT-OSS!" + bytes(data[12:]))
    with pytest.raises(ValueError, match="magic"):
        loaders.read_modelbin_header(bad)
    cut = tmp_path / "cut.bin"
    cut.write_bytes(bytes(data[:-100]))
    with pytest.raises(ValueError, match="truncated"):
        loaders.load_modelbin_moe(cut)


def _checkpoint(layer_data, l):
    """Original GPT-OSS checkpoint tensors of one layer (blocks [E, rows, G, 16], raw e8m0)."""
    nm = loaders.gptoss_moe_tensor_names(l)
    d = layer_data
    bits = synth.f32_to_bf16_bits
    return {
        nm["w1b"]: ("U8", d.w1_blocks.reshape(E, 2 * F, D // 32, 16)),
        nm["w1s"]: ("U8", ((d.w1_scales.astype(np.int32) - d.ue8_offset) % 256).astype(np.uint8)),
        nm["b1"]: ("BF16", bits(d.b1_f32)),
        nm["w2b"]: ("U8", d.w2_blocks.reshape(E, D, F // 32, 16)),
        nm["w2s"]: ("U8", ((d.w2_scales.astype(np.int32) - d.ue8_offset) % 256).astype(np.uint8)),
        nm["b2"]: ("BF16", bits(d.b2_f32)),
        nm["gw"]: ("BF16", bits(d.router_w_f32)),
        nm["gb"]: ("BF16", bits(d.router_b_f32)),
        nm["norm"]: ("BF16", bits(d.gamma_f32)),
    }


def test_safetensors_round_trip(tmp_path):
    src = _layers(2)
    tensors = {}
    for l, d in enumerate(src):
        tensors.update(_checkpoint(d, l))
    tensors["block.0.attn.norm.scale"] = ("BF16", np.zeros(D, np.uint16))  # unrelated tensors are ignored
    path = tmp_path / "model.safetensors"
    loaders.write_safetensors(path, tensors)
    st = loaders.read_safetensors(path)
    assert st["block.1.mlp.mlp1_weight.blocks"][1].shape == (E, 2 * F, D // 32, 16)
    for l, d in enumerate(src):
        got = loaders.load_safetensors_moe(path, l, experts_per_token=K)
        assert got.ue8_offset == 0 and got.gate_up_layout == "interleaved" and got.dtype == "bf16"
        _same_layer(d, got)


def test_safetensors_missing_tensor(tmp_path):
    tensors = _checkpoint(_layers(1)[0], 0)
    del tensors["block.0.mlp.gate.bias"]
    path = tmp_path / "m.safetensors"
    loaders.write_safetensors(path, tensors)
    with pytest.raises(KeyError, match="gate.bias"):
        loaders.load_safetensors_moe(path, 0)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["modelbin", "modelbin_halves", "safetensors"])
def test_loaded_layer_forward_matches(tmp_path, oracle, fmt):
    """A layer read back from disk gives the same outputs, bit for bit, as the in-memory layer it
    was written from (read with the same gate_up row pairing), and agrees with the oracle.  A
    model.bin loads with the checkpoints' interleaved pairing by default; "halves" is the opt-in
    pairing of the reference kernel."""
    from burnext_amd import moe
    src = _layers(1)[0]
    if fmt == "modelbin":
        path = tmp_path / "model.bin"
        loaders.write_modelbin(path, _header(1), [src])
        got = loaders.load_modelbin_moe(path)[0]
        assert got.gate_up_layout == "interleaved"
    elif fmt == "modelbin_halves":
        path = tmp_path / "model.bin"
        loaders.write_modelbin(path, _header(1), [src])
        got = loaders.load_modelbin_moe(path, gate_up_layout="halves")[0]
        src = dataclasses.replace(src, gate_up_layout="halves")
    else:
        path = tmp_path / "model.safetensors"
        loaders.write_safetensors(path, _checkpoint(src, 0))
        got = loaders.load_safetensors_moe(path, 0, experts_per_token=K)
    x = synth.make_tokens(40, D, seed=2, dtype="bf16")
    outs = []
    for data in (src, got):
        layer = moe.MoeLayer(data)
        outs.append(layer.forward(moe.to_device_x(x, "bf16")).float().cpu().numpy())
        torch.cuda.synchronize()
        layer.close()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    y_ref, _, _ = oracle.moe_forward(got, x)
    assert oracle.max_abs_rel(outs[1], y_ref) <= 2e-2
