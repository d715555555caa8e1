"""Synthetic routed-expert checkpoints for the loader tests: seeded fp32 expert weights,
quantized by the oracle into the checkpoint formats (MXFP4: int8-packed e2m1 + E8M0 per 32;
FP8 block: e4m3 + fp32 128x128 scales) and written as safetensors shards under the names of
DeepSeek-V4 ("dsv4": layers.L.ffn.experts.E.w1.weight / .scale) or Hugging Face ("hf":
model.layers.L.mlp.experts.E.gate_proj.weight / .weight_scale_inv), with non-expert tensors
(attention, router, shared experts) and an MTP layer's experts beside them."""

import os

import numpy as np
import torch

from oracle import formats as F

NAMES = {
    "dsv4": ("layers.{l}.ffn.experts.{e}.{p}.{k}", {"gate": "w1", "up": "w3", "down": "w2"},
             {"weight": "weight", "scale": "scale"}),
    "hf": ("model.layers.{l}.mlp.experts.{e}.{p}.{k}", {"gate": "gate_proj", "up": "up_proj", "down": "down_proj"},
           {"weight": "weight", "scale": "weight_scale_inv"}),
}


def quantize(w: np.ndarray, fmt: str):
    """fp32 [N, K] -> (checkpoint weight tensor, checkpoint scale tensor)."""
    if fmt == "mxfp4":
        codes, scales = F.mx_quantize(w, "e2m1")
        return (torch.from_numpy(F.pack_fp4(codes)).view(torch.int8),
                torch.from_numpy(scales).view(torch.float8_e8m0fnu))
    codes, s = F.fp8_block_quantize_2d(w)
    return torch.from_numpy(codes).view(torch.float8_e4m3fn), torch.from_numpy(s)


def expert_fp32(layer: int, expert: int, hidden: int, inter: int, seed: int):
    g = np.random.default_rng(seed * 100003 + layer * 1009 + expert)
    w13 = (g.standard_normal((2 * inter, hidden)) * 0.02).astype(np.float32)
    w2 = (g.standard_normal((hidden, inter)) * 0.02).astype(np.float32)
    return w13, w2


def write_checkpoint(path, *, layers, num_experts, hidden, inter, fmt, naming, seed=0, shards=3):
    """Writes the shards; returns (files, {layer: (w13 [E, 2I, H], w2 [E, H, I]) fp32 of every
    expert}). Layer ``layers`` (one past the last) is an MTP layer with experts of its own."""
    from safetensors.torch import save_file

    fmt_name, proj, kind = NAMES[naming]
    tensors, logical = {}, {}
    for l in range(layers + 1):
        w13s, w2s = [], []
        for e in range(num_experts):
            w13, w2 = expert_fp32(l, e, hidden, inter, seed)
            w13s.append(w13)
            w2s.append(w2)
            for p, w in (("gate", w13[:inter]), ("up", w13[inter:]), ("down", w2)):
                wt, sc = quantize(w, fmt)
                tensors[fmt_name.format(l=l, e=e, p=proj[p], k=kind["weight"])] = wt
                tensors[fmt_name.format(l=l, e=e, p=proj[p], k=kind["scale"])] = sc
        prefix = "model.layers" if naming == "hf" else "layers"
        tensors[f"{prefix}.{l}.self_attn.q_proj.weight"] = torch.zeros(8, hidden, dtype=torch.bfloat16)
        tensors[f"{prefix}.{l}.mlp.gate.weight"] = torch.zeros(num_experts, hidden, dtype=torch.float32)
        tensors[f"{prefix}.{l}.mlp.shared_experts.gate_proj.weight"] = torch.zeros(inter, hidden, dtype=torch.bfloat16)
        if l < layers:
            logical[l] = (np.stack(w13s), np.stack(w2s))
    names = sorted(tensors)
    files = []
    for s in range(shards):
        f = os.path.join(path, f"model-{s + 1:05d}-of-{shards:05d}.safetensors")
        save_file({n: tensors[n].contiguous() for n in names[s::shards]}, f)
        files.append(f)
    return files, logical


def dequantized(w: np.ndarray, fmt: str) -> np.ndarray:
    """The weights the checkpoint holds, as fp32 (what the oracle computes with)."""
    if fmt == "mxfp4":
        codes, scales = F.mx_quantize(w, "e2m1")
        return F.mx_dequantize(codes, scales, "e2m1")
    codes, s = F.fp8_block_quantize_2d(w)
    return F.fp8_block_dequantize_2d(codes, s)
