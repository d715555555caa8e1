"""Checkpoint load of an FFN rank's routed experts: select by name, stack, repack on the GPU.

Selection follows ``python/sgl_asap_plugin/srt/model_loader/weight_utils.py`` (the whole
file): a role picks a filter before any byte is read, ``skip_routed_experts()`` for an
attention rank and ``read_routed_experts_only(experts, num_layers)`` for an FFN rank, and
``filtered_safetensors_iterator`` yields ``(name, tensor)`` of the kept tensors only, reading
a few shards ahead on a thread pool. A routed expert is ``.experts.<E>.`` in a name, its
decoder layer ``layers.<L>.`` (DeepSeek-V4's ``layers.3.ffn.experts.17.w1.weight``, Hugging
Face's ``model.layers.3.mlp.experts.17.gate_proj.weight``).

The reference hands the kept tensors to SGLang's FusedMoE weight loader. Here
``load_routed_experts`` groups them per layer and repacks each complete layer on the GPU
(``repack_mxfp4_experts`` / ``repack_fp8_block_experts``), bytes unchanged, as soon as its
last tensor arrives, so host memory holds at most the layers still incomplete. The format
follows the tensors: 1-byte packed e2m1 codes with an E8M0 scale per 32 (MXFP4, the ERNIE 5.5
and DeepSeek-V4 FP4 experts, ``srt/configs/model_config.py:3-7``) or e4m3 codes with fp32
128x128 block scales (FP8 block experts).
"""

from __future__ import annotations

import concurrent.futures
import os
import re
from collections import defaultdict, deque
from dataclasses import dataclass
from typing import Callable, Dict, Iterable, Iterator, Optional, Sequence, Tuple

import torch

_EXPERT = re.compile(r"\.experts\.(\d+)\.")
_LAYER = re.compile(r"(?:^|\.)layers\.(\d+)\.")
# the projection and tensor kind after ``.experts.<E>.``: DeepSeek-V4 names w1/w3/w2 with
# ``.scale``, Hugging Face gate/up/down_proj with ``.weight_scale_inv`` (or ``.weight_scale``)
_PROJ = {"w1": "gate", "gate_proj": "gate", "w3": "up", "up_proj": "up", "w2": "down", "down_proj": "down"}
_KIND = {"weight": "weight", "scale": "scale", "weight_scale_inv": "scale", "weight_scale": "scale"}
_TAIL = re.compile(r"\.experts\.\d+\.([A-Za-z0-9_]+)\.([A-Za-z_]+)$")

_keep: Optional[Callable[[str], bool]] = None  # the tensors this process reads; None: all


def skip_routed_experts() -> None:
    """Attention ranks: every tensor but the routed experts."""
    global _keep
    _keep = lambda name: _EXPERT.search(name) is None  # noqa: E731


def routed_expert_filter(experts: range, num_layers: int) -> Callable[[str], bool]:
    """True for a routed expert of ``experts`` in a decoder layer below ``num_layers`` (an MTP
    layer's experts, numbered past the decoder layers, are not read)."""

    def keep(name: str) -> bool:
        e, l = _EXPERT.search(name), _LAYER.search(name)
        return e is not None and l is not None and int(l.group(1)) < num_layers and int(e.group(1)) in experts

    return keep


def read_routed_experts_only(experts: range, num_layers: int) -> None:
    """FFN ranks: the routed experts in ``experts`` of the decoder layers, nothing else."""
    global _keep
    _keep = routed_expert_filter(experts, num_layers)


def keep_filter() -> Optional[Callable[[str], bool]]:
    return _keep


def reset_filter() -> None:
    global _keep
    _keep = None


def filtered_safetensors_iterator(files: Sequence[str], keep: Callable[[str], bool], *, max_workers: int = 4,
                                  disable_mmap: bool = False) -> Iterator[Tuple[str, torch.Tensor]]:
    """``(name, tensor)`` of the kept tensors of ``files``, file by file in order, names sorted
    within a file. Up to ``max_workers + 1`` files are read ahead on a thread pool; a tensor
    that ``keep`` rejects is never read."""
    import safetensors

    def read(path: str) -> Dict[str, torch.Tensor]:
        if disable_mmap:
            return _read_unmapped(path, keep)
        with safetensors.safe_open(path, framework="pt", device="cpu") as f:
            return {k: f.get_tensor(k) for k in f.keys() if keep(k)}

    todo = deque(files)
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, max_workers)) as pool:
        ahead = deque()
        while todo and len(ahead) < max_workers + 1:
            ahead.append(pool.submit(read, todo.popleft()))
        while ahead:
            tensors = ahead.popleft().result()
            if todo:
                ahead.append(pool.submit(read, todo.popleft()))
            for name in sorted(tensors):
                yield name, tensors.pop(name)


_ST_DTYPES = {
    "BOOL": torch.bool, "U8": torch.uint8, "I8": torch.int8, "I16": torch.int16, "I32": torch.int32,
    "I64": torch.int64, "F16": torch.float16, "BF16": torch.bfloat16, "F32": torch.float32,
    "F64": torch.float64, "F8_E4M3": torch.float8_e4m3fn, "F8_E5M2": torch.float8_e5m2,
    "F8_E8M0": torch.float8_e8m0fnu,
}


def _read_unmapped(path: str, keep: Callable[[str], bool]) -> Dict[str, torch.Tensor]:
    """The kept tensors of one safetensors file, read with plain reads (no mmap): the 8-byte
    little-endian header size, the JSON header, then each kept tensor's byte range."""
    import json
    import struct

    out = {}
    with open(path, "rb") as f:
        (size,) = struct.unpack("<Q", f.read(8))
        header = json.loads(f.read(size))
        base = 8 + size
        for name, meta in header.items():
            if name == "__metadata__" or not keep(name):
                continue
            if meta["dtype"] not in _ST_DTYPES:
                raise ValueError(f"{path}: tensor {name} has dtype {meta['dtype']}, not one this loader reads")
            lo, hi = meta["data_offsets"]
            f.seek(base + lo)
            buf = bytearray(f.read(hi - lo))
            raw = torch.frombuffer(buf, dtype=torch.uint8) if buf else torch.empty(0, dtype=torch.uint8)
            out[name] = raw.view(_ST_DTYPES[meta["dtype"]]).reshape(meta["shape"])
    return out


def expert_tensor(name: str) -> Optional[Tuple[int, int, str, str]]:
    """(layer, expert, projection "gate"/"up"/"down", kind "weight"/"scale") of a routed-expert
    tensor name, or None for any other tensor."""
    e, l, t = _EXPERT.search(name), _LAYER.search(name), _TAIL.search(name)
    if e is None or l is None or t is None or t.group(1) not in _PROJ or t.group(2) not in _KIND:
        return None
    return int(l.group(1)), int(e.group(1)), _PROJ[t.group(1)], _KIND[t.group(2)]


@dataclass
class LayerTensors:
    """One layer's local experts as the checkpoint holds them, stacked (CPU tensors):
    w13 [E, 2I, H/2 or H] codes with rows [gate; up], s13 its scales, w2 / s2 the down
    projection's. ``fmt`` is "mxfp4" or "fp8_block"."""

    fmt: str
    w13: torch.Tensor
    s13: torch.Tensor
    w2: torch.Tensor
    s2: torch.Tensor


def _format_of(weight: torch.Tensor, scale: torch.Tensor, name: str) -> str:
    if weight.dtype == torch.float8_e4m3fn and scale.dtype == torch.float32:
        return "fp8_block"
    if weight.element_size() == 1 and weight.dtype != torch.float8_e4m3fn and scale.element_size() == 1:
        return "mxfp4"
    raise ValueError(f"{name}: weight {weight.dtype} with scale {scale.dtype} is neither MXFP4 "
                     "(1-byte packed e2m1 + E8M0) nor FP8 block (e4m3 + fp32)")


def stack_layer(parts: Dict[Tuple[int, str, str], torch.Tensor], local: range, layer: int) -> LayerTensors:
    """The per-expert tensors of one layer, keyed (expert, projection, kind), as LayerTensors.
    Raises ValueError when a tensor is missing or the experts disagree in format or shape."""
    missing = [(e, p, k) for e in local for p in ("gate", "up", "down") for k in ("weight", "scale")
               if (e, p, k) not in parts]
    if missing:
        raise ValueError(f"layer {layer}: missing routed-expert tensors {missing[:6]}{' ...' if len(missing) > 6 else ''}")
    fmt = _format_of(parts[(local.start, "gate", "weight")], parts[(local.start, "gate", "scale")], f"layer {layer}")
    w13, s13, w2, s2 = [], [], [], []
    for e in local:
        g = {(p, k): parts[(e, p, k)] for p in ("gate", "up", "down") for k in ("weight", "scale")}
        if _format_of(g[("gate", "weight")], g[("gate", "scale")], f"layer {layer} expert {e}") != fmt:
            raise ValueError(f"layer {layer}: expert {e} is not {fmt} like expert {local.start}")
        if g[("gate", "weight")].shape != g[("up", "weight")].shape or g[("gate", "scale")].shape != g[("up", "scale")].shape:
            raise ValueError(f"layer {layer} expert {e}: gate and up projections differ in shape")
        w13.append(torch.cat([g[("gate", "weight")], g[("up", "weight")]]))
        s13.append(torch.cat([g[("gate", "scale")], g[("up", "scale")]]))
        w2.append(g[("down", "weight")])
        s2.append(g[("down", "scale")])
    try:
        return LayerTensors(fmt, torch.stack(w13), torch.stack(s13), torch.stack(w2), torch.stack(s2))
    except RuntimeError as exc:
        raise ValueError(f"layer {layer}: local experts differ in shape ({exc})") from None


def pack_layer(t: LayerTensors, device=None):
    """LayerTensors -> ExpertWeights on ``device`` (the kernel's layout, bytes unchanged)."""
    from .moe.experts import repack_fp8_block_experts, repack_mxfp4_experts

    repack = repack_mxfp4_experts if t.fmt == "mxfp4" else repack_fp8_block_experts
    return repack(t.w13, t.s13, t.w2, t.s2, device=device)


def group_routed_experts(named: Iterable[Tuple[str, torch.Tensor]], local: range,
                         on_layer: Callable[[int, LayerTensors], None]) -> None:
    """Group routed-expert tensors of ``local`` by layer; call ``on_layer`` once per layer as
    soon as its 6 tensors per expert are all there. Other tensors are ignored; layers still
    incomplete at the end raise ValueError."""
    pending: Dict[int, Dict[Tuple[int, str, str], torch.Tensor]] = defaultdict(dict)
    need = 6 * len(local)
    for name, tensor in named:
        key = expert_tensor(name)
        if key is None or key[1] not in local:
            continue
        layer, expert, proj, kind = key
        parts = pending[layer]
        if (expert, proj, kind) in parts:
            raise ValueError(f"{name}: a second tensor for layer {layer} expert {expert} {proj} {kind}")
        parts[(expert, proj, kind)] = tensor
        if len(parts) == need:
            on_layer(layer, stack_layer(pending.pop(layer), local, layer))
    for layer, parts in pending.items():
        stack_layer(parts, local, layer)  # raises, naming what is missing


def load_routed_experts(files: Sequence[str], local: range, num_layers: int, *, device=None,
                        max_workers: int = 4) -> Dict[int, "object"]:
    """{layer: ExpertWeights} of the routed experts ``local`` in the decoder layers below
    ``num_layers``, read from safetensors ``files`` (only those tensors are read) and repacked
    on ``device`` layer by layer."""
    files = [os.fspath(f) for f in files]
    out = {}
    named = filtered_safetensors_iterator(files, routed_expert_filter(local, num_layers), max_workers=max_workers)
    group_routed_experts(named, local, lambda layer, t: out.__setitem__(layer, pack_layer(t, device)))
    return out
