"""Writes the committed fixtures of tests/golden/.

* mxfp4_dequant_kats.json -- the two known answers of the reference's
  tests/mxfp4_dequant_tests.rs:4-25 (blocks [0x10, 0x21] with scale 127 and 128), as data.
* tiny_c1.npz -- config 1 (T=16, D=F=256, E=k=2, f32, seed 0) inputs from burnext_amd.synth and the
  oracle's outputs (logits, top-k, weights, layer output for both gate_up layouts).
* decode_c2_routing.npz -- config 2 (T=8, D=2880, E=32, k=4, bf16, seed 0) routing outputs.

Run from the repository root:  python tests/golden/gen_golden.py
"""
import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT / "burn-extended_amd"))
sys.path.insert(0, str(ROOT / "oracle"))

import oracle as O  # noqa: E402
from burnext_amd import synth  # noqa: E402


def main():
    kats = {"source": "reference tests/mxfp4_dequant_tests.rs:4-25",
            "blocks": [0x10, 0x21], "blocks_shape": [1, 2], "scales_shape": [1],
            "cases": [{"scale": 127, "expect": [0.0, 0.5, 0.5, 1.0]}, {"scale": 128, "expect": [0.0, 1.0, 1.0, 2.0]}]}
    (HERE / "mxfp4_dequant_kats.json").write_text(json.dumps(kats, indent=1) + "\n")

    L = synth.make_layer(256, 256, 2, 2, seed=0, dtype="f32")
    x = synth.make_tokens(16, 256, seed=0, dtype="f32")
    lg = O.route_logits(x, L.router_w_f32, L.router_b_f32, None, L.rms_eps, True)
    idx, w = O.topk_softmax(lg, 2)
    y_int, _, _ = O.moe_forward(L, x, layout="interleaved")
    y_hal, _, _ = O.moe_forward(L, x, layout="halves")
    np.savez_compressed(HERE / "tiny_c1.npz", x=x, w1_blocks=L.w1_blocks, w1_scales=L.w1_scales,
                        w2_blocks=L.w2_blocks, w2_scales=L.w2_scales, b1=L.b1_f32, b2=L.b2_f32,
                        router_w=L.router_w_f32, router_b=L.router_b_f32, logits=lg, topk_idx=idx, topk_w=w,
                        y_interleaved=y_int, y_halves=y_hal)

    L2 = synth.make_layer(2880, 2880, 32, 4, seed=0, dtype="bf16")
    x2 = synth.make_tokens(8, 2880, seed=0, dtype="bf16")
    lg2 = O.route_logits(x2, L2.router_w_f32, L2.router_b_f32, None, L2.rms_eps, True)
    idx2, w2 = O.topk_softmax(lg2, 4)
    np.savez_compressed(HERE / "decode_c2_routing.npz", x_bf16_bits=synth.f32_to_bf16_bits(x2),
                        router_w_bf16_bits=L2.router_w_bits, logits=lg2, topk_idx=idx2, topk_w=w2)
    print("wrote", sorted(p.name for p in HERE.iterdir() if p.suffix in (".json", ".npz")))


if __name__ == "__main__":
    main()
