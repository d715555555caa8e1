"""Writes tests/golden/tiny_mxfp4.npz: the tiny MoE layer (hidden 256, inter 128, 8 experts
all local, top-2, 64 tokens, seed 0) as inputs, MXFP4 expert weights (e2m1 codes packed two
per byte, element 2i in the low nibble, plus UE8M0 scales per 32 along K) and the oracle's
routing and bf16 output.

The reference holds no golden vectors for this path, so the fixture is the oracle's output
on the seeded workload; tests/test_golden.py checks that the oracle still reproduces it and
tests/test_gpu_golden.py runs the HIP path on the stored codes.

    python tests/golden/make_tiny.py
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "sgl-afd-plugin_amd")]

from oracle import experts as OX  # noqa: E402
from oracle import formats as F  # noqa: E402
from oracle import routing as R  # noqa: E402
from sgl_asap_amd import workloads as W  # noqa: E402

PATH = os.path.join(HERE, "tiny_mxfp4.npz")


def build():
    s = W.SHAPES["tiny"]
    gen = W.generator("cpu", 0)
    x = W.tokens(s.tokens, s.hidden, gen, "cpu")
    ids, w = W.route_uniform(s.tokens, s.num_experts, s.top_k, gen, "cpu")
    w13, w2 = W.expert_weights(s.num_local, s.hidden, s.inter, gen, "cpu")
    c13, s13 = F.mx_quantize(w13.numpy(), "e2m1")
    c2, s2 = F.mx_quantize(w2.numpy(), "e2m1")
    w13d, w2d = F.mx_dequantize(c13, s13, "e2m1"), F.mx_dequantize(c2, s2, "e2m1")
    out = OX.moe_ffn(x, ids.numpy(), w.numpy(), w13d, w2d, 0, act="mxfp8")
    r = R.route(ids.numpy(), 0, s.num_local, 128)
    return {
        "x_bits": x.view(torch.int16).numpy().view(np.uint16),
        "topk_ids": ids.numpy(),
        "topk_weights": w.numpy(),
        "w13_packed": F.pack_fp4(c13),
        "w13_scales": s13,
        "w2_packed": F.pack_fp4(c2),
        "w2_scales": s2,
        "counts": r["counts"],
        "padded_offsets": r["padded_offsets"],
        "sorted_pairs": r["sorted_pairs"],
        "pair_pos": r["pair_pos"],
        "out_bits": out,
        "shape": np.array([s.hidden, s.inter, s.num_experts, s.num_local, s.top_k, s.tokens], dtype=np.int64),
    }


if __name__ == "__main__":
    np.savez_compressed(PATH, **build())
    print(PATH, os.path.getsize(PATH), "bytes")
