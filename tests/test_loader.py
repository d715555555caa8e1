"""CPU: the checkpoint expert loader's name filters (the semantics stated by
srt/model_loader/weight_utils.py of the reference), its safetensors iterator, and the
grouping of one layer's experts into the stacked checkpoint tensors."""

import numpy as np
import pytest
import torch

import ckpt
from oracle import formats as F
from sgl_asap_amd import loader as LD

NAMES = [
    # (name, routed expert (layer, expert) or None)
    ("layers.3.ffn.experts.17.w1.weight", (3, 17)),
    ("model.layers.3.mlp.experts.17.gate_proj.weight", (3, 17)),
    ("model.layers.12.mlp.experts.5.down_proj.weight_scale_inv", (12, 5)),
    ("layers.1.ffn.experts.40.w2.scale", (1, 40)),
    ("model.layers.3.mlp.gate.weight", None),
    ("model.layers.3.mlp.shared_experts.gate_proj.weight", None),
    ("model.layers.3.self_attn.q_proj.weight", None),
    ("model.embed_tokens.weight", None),
]


@pytest.mark.parametrize("name,routed", NAMES)
def test_filters(name, routed):
    try:
        LD.skip_routed_experts()
        assert LD.keep_filter()(name) == (routed is None)
        LD.read_routed_experts_only(range(16, 48), num_layers=4)
        want = routed is not None and routed[0] < 4 and 16 <= routed[1] < 48
        assert LD.keep_filter()(name) == want
    finally:
        LD.reset_filter()
    assert LD.keep_filter() is None


def test_mtp_layer_experts_not_read():
    keep = LD.routed_expert_filter(range(0, 64), num_layers=3)
    assert keep("layers.2.ffn.experts.0.w1.weight")
    assert not keep("layers.3.ffn.experts.0.w1.weight")  # layer 3 = the MTP layer
    assert not keep("layers.30.ffn.experts.0.w1.weight")  # "layers.3" is not a prefix match


@pytest.mark.parametrize("name,parsed", [
    ("layers.3.ffn.experts.17.w1.weight", (3, 17, "gate", "weight")),
    ("layers.3.ffn.experts.17.w3.scale", (3, 17, "up", "scale")),
    ("model.layers.0.mlp.experts.2.down_proj.weight_scale_inv", (0, 2, "down", "scale")),
    ("model.layers.0.mlp.experts.2.up_proj.weight_scale", (0, 2, "up", "scale")),
    ("model.layers.0.mlp.experts.2.up_proj.bias", None),
    ("model.layers.0.mlp.shared_experts.up_proj.weight", None),
])
def test_expert_tensor_names(name, parsed):
    assert LD.expert_tensor(name) == parsed


def _checkpoint(tmp_path, fmt, naming, **kw):
    args = dict(layers=2, num_experts=6, hidden=256, inter=128, fmt=fmt, naming=naming, seed=1)
    args.update(kw)
    return ckpt.write_checkpoint(str(tmp_path), **args)


@pytest.mark.parametrize("workers,mmap_off", [(1, False), (4, False), (2, True)])
def test_iterator_reads_only_kept_tensors(tmp_path, workers, mmap_off):
    files, _ = _checkpoint(tmp_path, "mxfp4", "hf")
    keep = LD.routed_expert_filter(range(2, 4), num_layers=2)
    got = list(LD.filtered_safetensors_iterator(files, keep, max_workers=workers, disable_mmap=mmap_off))
    names = [n for n, _ in got]
    assert len(names) == 2 * 2 * 6  # 2 layers x 2 experts x (3 weights + 3 scales)
    assert all(keep(n) for n in names)
    # file by file, names sorted within a file: the names of each shard form a sorted run
    from safetensors import safe_open

    expect = []
    for f in files:
        with safe_open(f, framework="pt") as h:
            expect += sorted(k for k in h.keys() if keep(k))
    assert names == expect


@pytest.mark.parametrize("fmt", ["mxfp4", "fp8_block"])
@pytest.mark.parametrize("naming", ["dsv4", "hf"])
def test_group_layers_stacks_gate_up(tmp_path, fmt, naming):
    files, logical = _checkpoint(tmp_path, fmt, naming)
    local = range(2, 5)
    layers = {}
    named = LD.filtered_safetensors_iterator(files, LD.routed_expert_filter(local, 2))
    LD.group_routed_experts(named, local, lambda l, t: layers.__setitem__(l, t))
    assert sorted(layers) == [0, 1]
    for l, t in layers.items():
        assert t.fmt == fmt
        w13, w2 = logical[l][0][local.start:local.stop], logical[l][1][local.start:local.stop]
        if fmt == "mxfp4":
            c13, s13 = F.mx_quantize(w13, "e2m1")
            c2, s2 = F.mx_quantize(w2, "e2m1")
            assert np.array_equal(t.w13.view(torch.uint8).numpy(), F.pack_fp4(c13))
            assert np.array_equal(t.s13.view(torch.uint8).numpy(), s13)
            assert np.array_equal(t.w2.view(torch.uint8).numpy(), F.pack_fp4(c2))
            assert np.array_equal(t.s2.view(torch.uint8).numpy(), s2)
        else:
            # the 128x128 blocks of gate and up never straddle (I % 128 == 0): quantizing the
            # stacked [gate; up] gives the per-projection codes and scales
            c13, s13 = F.fp8_block_quantize_2d(w13)
            c2, s2 = F.fp8_block_quantize_2d(w2)
            assert np.array_equal(t.w13.view(torch.uint8).numpy(), c13)
            assert np.array_equal(t.s13.numpy().view(np.uint32), s13.view(np.uint32))
            assert np.array_equal(t.w2.view(torch.uint8).numpy(), c2)
            assert np.array_equal(t.s2.numpy().view(np.uint32), s2.view(np.uint32))


def test_missing_duplicate_and_mixed_tensors_raise():
    def parts(fmt):
        wt, sc = ckpt.quantize(np.ones((128, 256), np.float32), fmt)
        return wt, sc

    mx, fp8 = parts("mxfp4"), parts("fp8_block")
    named = []
    for e in (0, 1):
        for p in ("w1", "w3", "w2"):
            src = mx if e == 0 else fp8
            named += [(f"layers.0.ffn.experts.{e}.{p}.weight", src[0]), (f"layers.0.ffn.experts.{e}.{p}.scale", src[1])]
    with pytest.raises(ValueError, match="not mxfp4"):
        LD.group_routed_experts(named, range(0, 2), lambda l, t: None)
    with pytest.raises(ValueError, match="missing"):
        LD.group_routed_experts(named[:-1], range(0, 2), lambda l, t: None)
    with pytest.raises(ValueError, match="second tensor"):
        LD.group_routed_experts(named[:1] + named, range(0, 2), lambda l, t: None)
