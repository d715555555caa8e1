"""GPU: seeded random layer shapes against the oracle, across both weight formats and the
three activations, with token counts at and around the 128-row tile edge (1, 2, 127, 128,
129, ...), partial local expert ranges and top-k from 1 to 8; and shapes of 2048-4096 tokens
where every GEMM workgroup takes several tiles, with both tile walks and bf16 activations.
Same bars as test_gpu_moe."""

import random

import pytest

from test_gpu_moe import assert_close, run_case

pytestmark = pytest.mark.gpu

CASES = 24


def draw(case: int) -> dict:
    rng = random.Random(7000 + case)
    fmt = rng.choice(["mxfp4", "fp8_block"])
    num_experts = rng.choice([8, 16, 32, 64])
    num_local = rng.randint(1, min(num_experts, 24))
    spec = dict(
        fmt=fmt,
        hidden=256 * rng.randint(1, 6),
        inter=128 * rng.randint(1, 6),
        num_experts=num_experts,
        num_local=num_local,
        e_lo=rng.randint(0, num_experts - num_local),
        k=rng.randint(1, min(8, num_experts)),
        n=rng.choice([1, 2, 31, 64, 127, 128, 129, 255, 300, 777]),
        zipf=rng.choice([None, 1.2]) if fmt == "fp8_block" else None,
    )
    act = rng.choice(["silu", "situ", "limit"])
    if act == "situ":
        spec["situ"] = (rng.choice([0.5, 2.0]), rng.choice([0.25, 3.0]))
    if act == "limit":
        spec["swiglu_limit"] = rng.choice([0.3, 1.0])
    return spec


@pytest.mark.parametrize("case", range(CASES))
def test_random_layer(case):
    s = draw(case)
    extra = {k: s[k] for k in ("situ", "swiglu_limit") if k in s}
    experts, out, ref, parts, (x, ids, w) = run_case(
        s["hidden"], s["inter"], s["num_experts"], s["e_lo"], s["num_local"], s["k"], s["n"], s["fmt"],
        9000 + case, zipf=s["zipf"], **extra)
    assert_close(out, ref, ids.numpy(), range(s["e_lo"], s["e_lo"] + s["num_local"]))


MANY_TILE_CASES = 12


def draw_many_tiles(case: int) -> dict:
    """Shapes where every GEMM workgroup takes several tiles (hidden of 3 K stages and more
    runs the continuous-ring gate_up), with both tile walks, bf16 activations and the three
    activations."""
    rng = random.Random(8100 + case)
    num_experts = rng.choice([16, 32, 64])
    num_local = rng.randint(num_experts // 4, num_experts)
    return dict(
        fmt=rng.choice(["mxfp4", "fp8_block"]),
        hidden=256 * rng.randint(2, 12),
        inter=128 * rng.randint(2, 8),
        num_experts=num_experts,
        num_local=num_local,
        e_lo=rng.randint(0, num_experts - num_local),
        k=rng.randint(2, 8),
        n=rng.choice([2048, 3000, 4096]),
        zipf=rng.choice([None, 1.2]),
        walk=rng.choice(["static", "dynamic"]),
        act_format=rng.choice([None, None, "bf16"]),
        act=rng.choice(["silu", "silu", "situ", "limit"]),
    )


@pytest.mark.parametrize("case", range(MANY_TILE_CASES))
def test_random_layer_many_tiles(case):
    s = draw_many_tiles(case)
    extra = {"situ": dict(situ=(1.702, 7.0)), "limit": dict(swiglu_limit=7.0)}.get(s["act"], {})
    experts, out, ref, parts, (x, ids, w) = run_case(
        s["hidden"], s["inter"], s["num_experts"], s["e_lo"], s["num_local"], s["k"], s["n"], s["fmt"],
        9500 + case, zipf=s["zipf"], walk=s["walk"], act_format=s["act_format"], **extra)
    assert_close(out, ref, ids.numpy(), range(s["e_lo"], s["e_lo"] + s["num_local"]))
