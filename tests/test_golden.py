"""The committed tiny-layer fixture (tests/golden/tiny_mxfp4.npz) against the oracle and
the workload generator (CPU): the oracle must still reproduce the stored routing and
output from the stored inputs and MXFP4 codes, and the seeded generator the stored inputs."""

import os

import numpy as np
import torch

from oracle import experts as OX
from oracle import formats as F
from oracle import routing as R
from sgl_asap_amd import workloads as W

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "tiny_mxfp4.npz")


def load():
    with np.load(GOLDEN) as d:
        return {k: d[k] for k in d.files}


def test_fixture_shape_is_the_tiny_layer():
    g = load()
    s = W.SHAPES["tiny"]
    assert g["shape"].tolist() == [s.hidden, s.inter, s.num_experts, s.num_local, s.top_k, s.tokens]


def test_oracle_reproduces_fixture():
    g = load()
    x = torch.from_numpy(g["x_bits"].view(np.int16)).view(torch.bfloat16)
    w13 = F.mx_dequantize(F.unpack_fp4(g["w13_packed"]), g["w13_scales"], "e2m1")
    w2 = F.mx_dequantize(F.unpack_fp4(g["w2_packed"]), g["w2_scales"], "e2m1")
    out = OX.moe_ffn(x, g["topk_ids"], g["topk_weights"], w13, w2, 0, act="mxfp8")
    assert np.array_equal(out, g["out_bits"])
    r = R.route(g["topk_ids"], 0, 8, 128)
    for key in ("counts", "padded_offsets", "sorted_pairs", "pair_pos"):
        assert np.array_equal(r[key], g[key]), key


def test_generator_reproduces_fixture_inputs():
    g = load()
    s = W.SHAPES["tiny"]
    x, ids, w = W.job(s, seed=0)
    assert np.array_equal(x.view(torch.int16).numpy().view(np.uint16), g["x_bits"])
    assert np.array_equal(ids.numpy(), g["topk_ids"]) and np.array_equal(w.numpy(), g["topk_weights"])
