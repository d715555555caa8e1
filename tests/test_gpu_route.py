"""GPU parity: the HIP router's permutation is bit-exact with the oracle's stable routing."""

import ctypes

import numpy as np
import pytest
import torch

from gpu_util import dev, say
from oracle import routing as R
from sgl_asap_amd import _lib
from sgl_asap_amd.moe.experts import workspace_layout

pytestmark = pytest.mark.gpu


def _i32(ws, off, count):
    return ws[off : off + 4 * count].view(torch.int32).cpu().numpy()


def run_route(ids: np.ndarray, e_lo: int, num_local: int, fmt=_lib.AFD_W_MXFP4):
    """fmt: the weight format, which sets the segment padding (MXFP4: 128 rows, FP8 blocks with
    fp8 activations: 256)."""
    n, k = ids.shape
    cfg = _lib.AfdMoeCfg(256, 128, k, e_lo, num_local, fmt)
    L = workspace_layout(cfg, n)
    ws = torch.full((L["total"],), 0xAB, dtype=torch.uint8, device=dev())
    ids_d = torch.from_numpy(np.ascontiguousarray(ids, dtype=np.int32)).to(dev())
    _lib.call("afd_route", ids_d.data_ptr(), n, ctypes.byref(cfg), ws.data_ptr(), ws.numel(),
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    poff = _i32(ws, L["padded_offsets"], num_local + 1)
    np_pad = int(poff[-1])
    tiles = int(_i32(ws, L["num_tiles"], 1)[0])
    return {
        "counts": _i32(ws, L["counts"], num_local),
        "offsets": _i32(ws, L["offsets"], num_local + 1),
        "padded_offsets": poff,
        "sorted_pairs": _i32(ws, L["sorted_pairs"], np_pad),
        "pair_pos": _i32(ws, L["pair_pos"], n * k),
        "tile_expert": _i32(ws, L["tile_expert"], tiles),
        "num_tiles": tiles,
        "block_m": L["block_m"],
    }


def check(ids, e_lo, num_local, fmt=_lib.AFD_W_MXFP4):
    got = run_route(ids, e_lo, num_local, fmt)
    ref = R.route(ids, e_lo, num_local, got["block_m"])
    for key in ("counts", "offsets", "padded_offsets", "sorted_pairs", "pair_pos"):
        assert np.array_equal(got[key], ref[key]), key
    tiles = ref["padded_offsets"][-1] // got["block_m"]
    assert got["num_tiles"] == tiles
    expect_tiles = np.repeat(np.arange(num_local), np.diff(ref["padded_offsets"]) // got["block_m"])
    assert np.array_equal(got["tile_expert"], expect_tiles)


CASES = [
    # (n, k, num_experts, e_lo, num_local, seed)
    (1, 1, 8, 0, 8, 0),
    (1, 8, 256, 0, 64, 1),
    (64, 2, 8, 0, 8, 2),
    (300, 4, 32, 8, 16, 3),
    (1000, 8, 256, 64, 64, 4),
    (4097, 8, 256, 192, 64, 5),
    (16384, 8, 256, 0, 64, 6),
    (2048, 6, 64, 0, 64, 7),
    (777, 32, 256, 0, 256, 8),
    (131071, 8, 256, 0, 64, 9),  # the largest job a doorbell announces: 1M pairs, 128 chunks
    (131071, 1, 256, 0, 256, 10),
    # more small-job shapes: 8192 pairs, one more, all 256 experts local, one local expert
    (1024, 8, 256, 0, 64, 11),
    (1025, 8, 256, 0, 64, 12),
    (200, 32, 256, 0, 256, 13),
    (500, 3, 16, 5, 1, 14),
]


@pytest.mark.parametrize("n,k,num_experts,e_lo,num_local,seed", CASES)
def test_route_random(n, k, num_experts, e_lo, num_local, seed):
    say(f"route n={n} k={k} experts={num_experts} local=[{e_lo},{e_lo + num_local}) seed={seed}")
    g = torch.Generator().manual_seed(seed)
    scores = torch.rand(n, num_experts, generator=g)
    ids = torch.topk(scores, k, dim=1).indices.to(torch.int32).numpy()
    check(ids, e_lo, num_local)


def test_route_edge_cases():
    say("route edge cases")
    # nothing local
    check(np.full((50, 4), 200, dtype=np.int32), 0, 64)
    # every pair on one expert, duplicates inside a row (graph padding rows)
    check(np.full((333, 8), 5, dtype=np.int32), 0, 64)
    # ids just outside both ends of the local range, and negative ids
    ids = np.array([[63, 64, 127, 128], [-1, 64, 65, 0]] * 40, dtype=np.int32)
    check(ids, 64, 64)
    # n = 0
    got = run_route(np.zeros((0, 8), dtype=np.int32), 0, 64)
    assert got["num_tiles"] == 0 and not got["counts"].any()


@pytest.mark.parametrize("n,k,num_experts,e_lo,num_local,seed", [CASES[i] for i in (1, 3, 5, 7, 8, 9, 13, 14)])
def test_route_256_row_segments(n, k, num_experts, e_lo, num_local, seed):
    """The FP8-block layout (W8A8) pads every expert segment to 256 rows: the same permutation,
    its own padded offsets and tile table, bit-exact against the oracle with block_m 256."""
    say(f"route256 n={n} k={k} experts={num_experts} local=[{e_lo},{e_lo + num_local}) seed={seed}")
    g = torch.Generator().manual_seed(seed)
    scores = torch.rand(n, num_experts, generator=g)
    ids = torch.topk(scores, k, dim=1).indices.to(torch.int32).numpy()
    got = run_route(ids, e_lo, num_local, _lib.AFD_W_FP8_BLOCK)
    assert got["block_m"] == 256
    check(ids, e_lo, num_local, _lib.AFD_W_FP8_BLOCK)
