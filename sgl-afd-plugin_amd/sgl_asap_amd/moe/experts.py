"""The F-side per-layer expert runner: what ``FusedMoE`` is to the reference's FFN rank.

The reference's FFN rank calls ``self.experts[layer_id](x, StandardTopKOutput(w, ids, None))``
(``python/sgl_asap_plugin/srt/managers/scheduler.py:410-412``) on a FusedMoE whose local
experts are ``range(ep_rank * per_rank, (ep_rank + 1) * per_rank)`` (``scheduler.py:206-218``)
and gets a bf16 [n, hidden] partial sum over the local experts. ``AfdExperts`` keeps that
call contract and runs it as one gfx950 call, ``afd_moe_ffn`` (include/afd.h):

    quantize x -> route pairs to local experts -> grouped gate_up + SwiGLU -> grouped down
    -> top-k weighted finalize

Weights are packed once at load time on the GPU (``pack_mxfp4_experts`` /
``pack_fp8_block_experts``) into the kernel's layout; a workspace sized for ``n_max`` tokens
is allocated once per stream, so a call only enqueues kernels (the handler contract of
``python/sgl_asap_plugin/transport/server.py:8-9``) and can be captured in a HIP graph.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict, Optional

import torch

from .. import _lib
from .topk import format_is_standard

WEIGHT_FORMATS = {"mxfp4": _lib.AFD_W_MXFP4, "fp8_block": _lib.AFD_W_FP8_BLOCK}
MX_BLOCK, FP8_BLOCK = 32, 128


def _stream_handle(stream: Optional[torch.cuda.Stream] = None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


@dataclass
class ExpertWeights:
    """Packed weights of one layer's local experts (device tensors, kernel layout)."""

    fmt: str  # "mxfp4" or "fp8_block"
    num_local: int
    hidden: int
    inter: int
    w13: torch.Tensor
    s13: torch.Tensor
    w2: torch.Tensor
    s2: torch.Tensor

    def as_struct(self) -> _lib.AfdExpertWeights:
        def ptr(t):
            return t.data_ptr() if t.numel() else None

        return _lib.AfdExpertWeights(ptr(self.w13), ptr(self.s13), ptr(self.w2), ptr(self.s2))

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.w13, self.s13, self.w2, self.s2))


def _as_f32(w: torch.Tensor, device) -> torch.Tensor:
    return w.to(device=device, dtype=torch.float32).contiguous()


def pack_mxfp4_experts(w13: torch.Tensor, w2: torch.Tensor, device=None) -> ExpertWeights:
    """Quantize logical expert weights to MXFP4 in the kernel's tile-image layout, on the GPU.

    w13: [E, 2I, H] with rows [gate; up] (SGLang's w13 mapping, ``srt/models/deepseek_v4.py:132-137``);
    w2: [E, H, I]. Any float dtype. The reference's checkpoints hold the same number format
    (int8-packed e2m1 + E8M0 per 32, ``srt/configs/model_config.py:3-7``); the images carry
    the codes and the scales together (include/afd.h describes the layout).
    """
    device = torch.device(device or "cuda")
    e, two_i, h = w13.shape
    inter = two_i // 2
    if w2.shape != (e, h, inter):
        raise ValueError(f"w2 shape {tuple(w2.shape)} does not match w13 {tuple(w13.shape)}")
    a = _as_f32(w13, device)
    b = _as_f32(w2, device)
    img13 = torch.empty(e, two_i * (h // 2 + h // MX_BLOCK), dtype=torch.uint8, device=device)
    img2 = torch.empty(e, h * (inter // 2 + inter // MX_BLOCK), dtype=torch.uint8, device=device)
    none = torch.empty(0, dtype=torch.uint8, device=device)
    with torch.cuda.device(device):
        st = _stream_handle()
        _lib.call("afd_pack_mxfp4", a.data_ptr(), e, two_i, h, 1, img13.data_ptr(), st)
        _lib.call("afd_pack_mxfp4", b.data_ptr(), e, h, inter, 0, img2.data_ptr(), st)
    return ExpertWeights("mxfp4", e, h, inter, img13, none, img2, none)


def pack_fp8_block_experts(w13: torch.Tensor, w2: torch.Tensor, device=None) -> ExpertWeights:
    """Quantize logical expert weights to e4m3 with fp32 128x128 block scales, on the GPU
    (the block-FP8 expert format of DeepGEMM / SGLang's Fp8MoEMethod)."""
    device = torch.device(device or "cuda")
    e, two_i, h = w13.shape
    inter = two_i // 2
    if w2.shape != (e, h, inter):
        raise ValueError(f"w2 shape {tuple(w2.shape)} does not match w13 {tuple(w13.shape)}")
    a = _as_f32(w13, device)
    b = _as_f32(w2, device)
    q13 = torch.empty(e, two_i, h, dtype=torch.uint8, device=device)
    s13 = torch.empty(e, two_i // FP8_BLOCK, h // FP8_BLOCK, dtype=torch.float32, device=device)
    q2 = torch.empty(e, h, inter, dtype=torch.uint8, device=device)
    s2 = torch.empty(e, h // FP8_BLOCK, inter // FP8_BLOCK, dtype=torch.float32, device=device)
    with torch.cuda.device(device):
        st = _stream_handle()
        _lib.call("afd_pack_fp8_block", a.data_ptr(), e, two_i, h, 1, q13.data_ptr(), s13.data_ptr(), st)
        _lib.call("afd_pack_fp8_block", b.data_ptr(), e, h, inter, 0, q2.data_ptr(), s2.data_ptr(), st)
    return ExpertWeights("fp8_block", e, h, inter, q13, s13, q2, s2)


def _bytes_on(t: torch.Tensor, device) -> torch.Tensor:
    """A 1-byte-element tensor (uint8 / int8 / float8 codes) as contiguous uint8 on device."""
    if t.element_size() != 1:
        raise TypeError(f"expected 1-byte codes, got {t.dtype}")
    return t.contiguous().view(torch.uint8).to(device)


def repack_mxfp4_experts(w13: torch.Tensor, s13: torch.Tensor, w2: torch.Tensor, s2: torch.Tensor,
                         device=None) -> ExpertWeights:
    """Already-quantized MXFP4 experts (a checkpoint's int8-packed e2m1 codes and E8M0 scales,
    ``srt/configs/model_config.py:3-7``) into the kernel's tile images, bytes unchanged.

    w13: [E, 2I, H/2] codes with rows [gate; up], s13: [E, 2I, H/32]; w2: [E, H, I/2],
    s2: [E, H, I/32]. Any 1-byte dtypes (uint8, int8, float8_e8m0fnu)."""
    device = torch.device(device or "cuda")
    e, two_i, hb = w13.shape
    h, inter = hb * 2, two_i // 2
    want = {"s13": (e, two_i, h // MX_BLOCK), "w2": (e, h, inter // 2), "s2": (e, h, inter // MX_BLOCK)}
    for name, t in (("s13", s13), ("w2", w2), ("s2", s2)):
        if tuple(t.shape) != want[name]:
            raise ValueError(f"{name} shape {tuple(t.shape)}, expected {want[name]} for w13 {tuple(w13.shape)}")
    c13, c2 = _bytes_on(w13, device), _bytes_on(w2, device)
    sc13, sc2 = _bytes_on(s13, device), _bytes_on(s2, device)
    img13 = torch.empty(e, two_i * (h // 2 + h // MX_BLOCK), dtype=torch.uint8, device=device)
    img2 = torch.empty(e, h * (inter // 2 + inter // MX_BLOCK), dtype=torch.uint8, device=device)
    none = torch.empty(0, dtype=torch.uint8, device=device)
    with torch.cuda.device(device):
        st = _stream_handle()
        _lib.call("afd_repack_mxfp4", c13.data_ptr(), sc13.data_ptr(), e, two_i, h, 1, img13.data_ptr(), st)
        _lib.call("afd_repack_mxfp4", c2.data_ptr(), sc2.data_ptr(), e, h, inter, 0, img2.data_ptr(), st)
    return ExpertWeights("mxfp4", e, h, inter, img13, none, img2, none)


def repack_fp8_block_experts(w13: torch.Tensor, s13: torch.Tensor, w2: torch.Tensor, s2: torch.Tensor,
                             device=None) -> ExpertWeights:
    """Already-quantized FP8 block experts (e4m3 codes, fp32 128x128 block scales as
    checkpoints store them: the dequantized weight is code x scale) into the kernel's row
    order, bytes unchanged. w13: [E, 2I, H] rows [gate; up], s13: [E, 2I/128, H/128];
    w2: [E, H, I], s2: [E, H/128, I/128]."""
    device = torch.device(device or "cuda")
    e, two_i, h = w13.shape
    inter = two_i // 2
    want = {"s13": (e, two_i // FP8_BLOCK, h // FP8_BLOCK), "w2": (e, h, inter),
            "s2": (e, h // FP8_BLOCK, inter // FP8_BLOCK)}
    for name, t in (("s13", s13), ("w2", w2), ("s2", s2)):
        if tuple(t.shape) != want[name]:
            raise ValueError(f"{name} shape {tuple(t.shape)}, expected {want[name]} for w13 {tuple(w13.shape)}")
    c13, c2 = _bytes_on(w13, device), _bytes_on(w2, device)
    q13 = torch.empty(e, two_i, h, dtype=torch.uint8, device=device)
    q2 = torch.empty(e, h, inter, dtype=torch.uint8, device=device)
    with torch.cuda.device(device):
        st = _stream_handle()
        _lib.call("afd_repack_fp8_block", c13.data_ptr(), e, two_i, h, 1, q13.data_ptr(), st)
        _lib.call("afd_repack_fp8_block", c2.data_ptr(), e, h, inter, 0, q2.data_ptr(), st)
    s13 = s13.to(device=device, dtype=torch.float32).contiguous()
    s2 = s2.to(device=device, dtype=torch.float32).contiguous()
    return ExpertWeights("fp8_block", e, h, inter, q13, s13, q2, s2)


ACTIVATIONS = {"silu": _lib.AFD_ACT_SWIGLU, "situ": _lib.AFD_ACT_SITU}


# the fp8 activation format each weight format's GEMMs read by default
FP8_ACT = {"mxfp4": "mxfp8", "fp8_block": "fp8_1x128"}


def moe_cfg(
    weights: ExpertWeights,
    top_k: int,
    expert_lo: int,
    activation: str = "silu",
    gemm1_alpha: Optional[float] = None,
    gemm1_clamp_limit: Optional[float] = None,
    act_format: Optional[str] = None,
) -> _lib.AfdMoeCfg:
    """The C config of a layer. ``activation`` is FusedMoE's ("silu": SwiGLU; "situ": SiTU
    with ``gemm1_alpha`` = its beta and ``gemm1_clamp_limit`` = its linear_beta, as the
    reference's ERNIE 5.5 experts pass them, P/srt/models/ernie55.py:43-55). "silu" with a
    ``gemm1_clamp_limit`` L is SwiGLU with a limit, silu(min(gate, L)) * clamp(up, -L, L):
    DeepSeek-V4's ``swiglu_limit`` (P/srt/models/deepseek_v4.py:63). ``act_format``: the
    precision of the GEMMs' activations, the weight format's fp8 form by default ("mxfp8" for
    MXFP4, "fp8_1x128" for FP8 blocks, the MoE methods' default quantization) or "bf16" (W4A16
    for MXFP4 weights: the reference's humming experts, scripts/run_ep.sh:4, README.md:25;
    W8A16 for FP8 blocks)."""
    fp8 = FP8_ACT[weights.fmt]
    if act_format not in (None, fp8, "bf16"):
        raise ValueError(f"activation format {act_format!r} for {weights.fmt} weights "
                         f"(supported: {fp8!r}, 'bf16')")
    act_fmt = _lib.AFD_A_BF16 if act_format == "bf16" else _lib.AFD_A_FP8
    if activation not in ACTIVATIONS:
        raise NotImplementedError(f"activation {activation!r} (supported: {sorted(ACTIVATIONS)})")
    alpha = limit = 0.0
    code = ACTIVATIONS[activation]
    if activation == "silu" and gemm1_clamp_limit is not None:
        limit = float(gemm1_clamp_limit)
        if not 0.0 < limit < float("inf"):
            raise ValueError(f"the SwiGLU limit must be positive and finite, got {limit}")
        code = _lib.AFD_ACT_SWIGLU_LIMIT
    if activation == "situ":
        if gemm1_alpha is None or gemm1_clamp_limit is None:
            # the reference's message (P/srt/layers/quantization/mxfp4_flashinfer_trtllm_moe.py:110-113)
            raise ValueError(
                "SiTU needs the layer's gemm1_alpha (beta) and gemm1_clamp_limit (linear_beta)"
            )
        alpha, limit = float(gemm1_alpha), float(gemm1_clamp_limit)
        if not (0.0 < alpha < float("inf") and 0.0 < limit < float("inf")):
            raise ValueError(f"SiTU constants must be positive and finite, got {alpha}, {limit}")
    return _lib.AfdMoeCfg(
        weights.hidden, weights.inter, top_k, expert_lo, weights.num_local, WEIGHT_FORMATS[weights.fmt],
        code, alpha, limit, _lib.AFD_WALK_STATIC, act_fmt,
    )


TILE_WALKS = {"static": _lib.AFD_WALK_STATIC, "dynamic": _lib.AFD_WALK_DYNAMIC}

# activation formats of the expert call's input -> the weight format whose GEMMs read them
ACT_FORMATS = {"mxfp8": "mxfp4", "fp8_1x128": "fp8_block"}


def act_scale_shape(act: str, n: int, hidden: int):
    """Shape and dtype of the scales of n tokens in activation format ``act``: "mxfp8" has
    hidden/32 UE8M0 bytes per token (each 128-wide K stage's four as blocks 0, 2, 1, 3),
    "fp8_1x128" hidden/128 fp32."""
    if act == "mxfp8":
        return (n, hidden // 32), torch.uint8
    if act == "fp8_1x128":
        return (n, hidden // 128), torch.float32
    raise ValueError(f"activation format {act!r} (supported: {sorted(ACT_FORMATS)})")


def quant_act(act: str, x: torch.Tensor, q: Optional[torch.Tensor] = None, s: Optional[torch.Tensor] = None,
              stream: Optional[torch.cuda.Stream] = None):
    """afd_quant_act without a layer: bf16 x [n, H] -> (e4m3 codes uint8 [n, H], scales), the
    input of afd_moe_ffn_q for experts of the matching weight format. The quantizer reads only
    the hidden size and the weight format of its configuration, so an attention rank, which
    holds no expert weights, quantizes its rows before the arena copy with this."""
    if act not in ACT_FORMATS:
        raise ValueError(f"activation format {act!r} (supported: {sorted(ACT_FORMATS)})")
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise TypeError(f"quant_act takes bf16 [n, H] activations, got {x.dtype} {tuple(x.shape)}")
    n, hidden = x.shape
    cfg = _lib.AfdMoeCfg(hidden, 128, 1, 0, 1, WEIGHT_FORMATS[ACT_FORMATS[act]], ACTIVATIONS["silu"], 0.0, 0.0)
    return _quant_act(cfg, act, x, q, s, stream)


def _quant_act(cfg, act, x, q, s, stream):
    x = x.contiguous()
    n, hidden = x.shape
    shape, dtype = act_scale_shape(act, n, hidden)
    q = torch.empty(n, hidden, dtype=torch.uint8, device=x.device) if q is None else q
    s = torch.empty(shape, dtype=dtype, device=x.device) if s is None else s
    if q.dtype != torch.uint8 or tuple(q.shape) != (n, hidden) or not q.is_contiguous():
        raise ValueError(f"q must be contiguous uint8 [{n}, {hidden}], got {q.dtype} {tuple(q.shape)}")
    if s.dtype != dtype or tuple(s.shape) != shape or not s.is_contiguous():
        raise ValueError(f"s must be contiguous {dtype} {shape}, got {s.dtype} {tuple(s.shape)}")
    if n > 0:
        _lib.call("afd_quant_act", ctypes.byref(cfg), x.data_ptr(), n, q.data_ptr(), s.data_ptr(),
                  _stream_handle(stream))
    return q, s


JOB_BYTES = ctypes.sizeof(_lib.AfdJob)

# Workspaces of the expert calls: one per (device, stream, size), shared by every layer whose
# calls need that size. Calls on one stream run in order, so a model's MoE layers (which
# usually share one size) use one buffer per stream instead of one each; calls on different
# streams get different buffers and may overlap. A buffer is never reallocated, and a graph
# runner keeps a workspace of its own, so pointers captured in HIP graphs stay valid.
_WORKSPACES: Dict[tuple, torch.Tensor] = {}


def stream_workspace(device: torch.device, stream_handle: int, nbytes: int) -> torch.Tensor:
    """The shared workspace of ``nbytes`` for calls on the stream ``stream_handle``."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, int(stream_handle), int(nbytes))
    ws = _WORKSPACES.get(key)
    if ws is None:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=torch.device("cuda", index))
        _WORKSPACES[key] = ws
    return ws


def release_workspaces() -> None:
    """Drop every shared workspace (after the device has finished the calls that used them)."""
    torch.cuda.synchronize()
    _WORKSPACES.clear()


def new_job_desc(device=None) -> torch.Tensor:
    """A zeroed device job descriptor (afd_job) for ``AfdExperts.call_job`` / ``set_job``."""
    return torch.zeros(JOB_BYTES, dtype=torch.uint8, device=device or "cuda")


def set_job(desc: torch.Tensor, *, ids: torch.Tensor, w: torch.Tensor, out: torch.Tensor,
            x: Optional[torch.Tensor] = None, xq: Optional[torch.Tensor] = None,
            xs: Optional[torch.Tensor] = None, stream: Optional[torch.cuda.Stream] = None) -> None:
    """Enqueue on ``stream`` (default: current) the write of one job into the descriptor
    (afd_job_set): bf16 ``x`` [n, H], or ``xq`` / ``xs`` from quant_act; int32 ``ids`` and fp32
    ``w`` [n, k]; bf16 ``out`` [n, H]. The tensors must stay alive until the calls that read
    the descriptor have run."""
    n = ids.shape[0]
    for name, t in (("ids", ids), ("w", w), ("out", out), ("x", x), ("xq", xq), ("xs", xs)):
        if t is not None and (not t.is_contiguous() or (t.dim() > 0 and t.shape[0] != n)):
            raise ValueError(f"{name} must be contiguous with {n} rows")
    if ids.dtype != torch.int32 or w.dtype != torch.float32 or out.dtype != torch.bfloat16:
        raise TypeError("ids int32, w float32 and out bf16 expected")
    if (x is None) == (xq is None or xs is None):
        raise ValueError("give either x or both xq and xs")

    def ptr(t):
        return t.data_ptr() if t is not None else None

    value = _lib.AfdJob(ptr(x), ptr(xq), ptr(xs), ptr(ids), ptr(w), ptr(out), n)
    _lib.call("afd_job_set", desc.data_ptr(), ctypes.byref(value), _stream_handle(stream))


def workspace_layout(cfg: _lib.AfdMoeCfg, n: int) -> dict:
    """afd_workspace_layout as a dict of byte offsets (plus np_max, block_m, max_tiles)."""
    out = _lib.AfdWsLayout()
    _lib.call("afd_workspace_layout", ctypes.byref(cfg), n, ctypes.byref(out))
    return {name: getattr(out, name) for name, _ in _lib.AfdWsLayout._fields_}


class AfdExperts(torch.nn.Module):
    """One MoE layer's local routed experts on one F rank.

    ``forward(hidden_states, topk_output)`` is the FusedMoE call of the reference's FFN
    rank: x bf16 [n, H], topk_output with ``topk_ids`` [n, k] (global ids) and
    ``topk_weights`` [n, k]; returns bf16 [n, H], the top-k-weighted sum over the local
    experts (rows with no local expert are 0). Enqueued on the current stream.

    ``activation``, ``gemm1_alpha`` and ``gemm1_clamp_limit`` are FusedMoE's (see
    ``moe_cfg``); ``swiglu_limit`` is DeepSeek-V4's FusedMoE argument, the clamp limit of
    its SwiGLU (P/srt/models/deepseek_v4.py:63).

    ``tile_walk`` (no counterpart in the reference): "static" gives each GEMM workgroup a
    fixed share of the tiles, best when the call has the GPU to itself; "dynamic" hands them
    out from per-XCD counters, for a GPU shared with other streams' kernels or parked stream
    waits (the FFN scheduler's setting). Results are identical bit for bit.

    ``act_format``: the activation precision of the GEMMs (``moe_cfg``): by default the
    weight format's fp8 form, which the call quantizes x and h to; "bf16" keeps x as it is
    and rounds h to bf16 (W4A16 for MXFP4 weights, W8A16 for FP8 blocks).
    """

    def __init__(
        self,
        num_experts: int,
        top_k: int,
        layer_id: int,
        local: range,
        weights: ExpertWeights,
        n_max: int = 16384,
        activation: str = "silu",
        gemm1_alpha: Optional[float] = None,
        gemm1_clamp_limit: Optional[float] = None,
        swiglu_limit: Optional[float] = None,
        tile_walk: str = "static",
        act_format: Optional[str] = None,
    ):
        super().__init__()
        if swiglu_limit is not None:  # DeepSeek-V4's FusedMoE argument: the SwiGLU clamp limit
            if activation != "silu" or (gemm1_clamp_limit is not None and gemm1_clamp_limit != swiglu_limit):
                raise ValueError("swiglu_limit applies to SwiGLU and is its gemm1_clamp_limit")
            gemm1_clamp_limit = swiglu_limit
        if len(local) != weights.num_local:
            raise ValueError(f"{len(local)} local experts but weights for {weights.num_local}")
        if not (0 <= local.start and local.stop <= num_experts):
            raise ValueError(f"local experts {local} outside [0, {num_experts})")
        self.num_experts, self.top_k, self.layer_id = num_experts, top_k, layer_id
        self.local = local
        self.hidden_size, self.intermediate_size = weights.hidden, weights.inter
        self.weights = weights
        self.n_max = n_max
        self.activation = activation
        self.cfg = moe_cfg(weights, top_k, local.start, activation, gemm1_alpha, gemm1_clamp_limit, act_format)
        self.tile_walk = tile_walk
        self.layout = workspace_layout(self.cfg, n_max)
        self._batch_bytes = {n_max: self.layout["total"]}  # workspace bytes per batch capacity
        self._wstruct = weights.as_struct()

    @property
    def tile_walk(self) -> str:
        return "dynamic" if self.cfg.tile_walk == _lib.AFD_WALK_DYNAMIC else "static"

    @tile_walk.setter
    def tile_walk(self, walk: str) -> None:
        if walk not in TILE_WALKS:
            raise ValueError(f"tile_walk must be one of {sorted(TILE_WALKS)}, got {walk!r}")
        self.cfg.tile_walk = TILE_WALKS[walk]

    def workspace(self, stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
        """The workspace of this layer's calls on ``stream`` (default: current): one per stream
        and size, shared with the other layers of that size (``stream_workspace``), so jobs
        on different streams can overlap while calls on one stream, which are ordered, share
        it."""
        s = stream if stream is not None else torch.cuda.current_stream()
        return stream_workspace(self.weights.w13.device, s.cuda_stream, self.layout["total"])

    def _topk(self, n: int, topk_output, device):
        if not format_is_standard(topk_output):
            raise RuntimeError(f"expected explicit top-k ids and weights, got {type(topk_output).__name__}")
        if n > self.n_max:
            raise ValueError(f"{n} tokens exceed n_max={self.n_max}")
        ids = topk_output.topk_ids
        w = topk_output.topk_weights
        if ids.shape != (n, self.top_k) or w.shape != (n, self.top_k):
            raise ValueError(f"top-k shapes {tuple(ids.shape)} / {tuple(w.shape)} for {n} tokens, k={self.top_k}")
        if ids.device != device or w.device != device:
            raise ValueError(f"top-k ids / weights on {ids.device} / {w.device}, activations on {device}")
        return ids.to(torch.int32).contiguous(), w.to(torch.float32).contiguous()

    def _out(self, out: Optional[torch.Tensor], n: int, device) -> torch.Tensor:
        """The caller's output tensor after checking it, or a new one: the kernels write
        n * hidden bf16 values through its data pointer."""
        if out is None:
            return torch.empty(n, self.hidden_size, dtype=torch.bfloat16, device=device)
        if out.dtype != torch.bfloat16 or tuple(out.shape) != (n, self.hidden_size):
            raise ValueError(f"out must be bf16 [{n}, {self.hidden_size}], got {out.dtype} {tuple(out.shape)}")
        if not out.is_contiguous() or out.device != torch.device(device):
            raise ValueError(f"out must be contiguous on {device}, got {out.device} "
                             f"{'contiguous' if out.is_contiguous() else 'strided'}")
        return out

    def forward(self, hidden_states: torch.Tensor, topk_output, out: Optional[torch.Tensor] = None):
        x = hidden_states
        if x.dtype != torch.bfloat16:
            raise TypeError(f"the expert path takes bf16 activations, got {x.dtype}")
        if x.dim() != 2 or x.shape[1] != self.hidden_size or not x.is_cuda:
            raise ValueError(f"x must be a device tensor [n, {self.hidden_size}], got {tuple(x.shape)} on {x.device}")
        n = x.shape[0]
        ids, w = self._topk(n, topk_output, x.device)
        x = x.contiguous()
        out = self._out(out, n, x.device)
        if n == 0:
            return out
        ws = self.workspace()
        _lib.call(
            "afd_moe_ffn",
            ctypes.byref(self.cfg),
            ctypes.byref(self._wstruct),
            x.data_ptr(),
            ids.data_ptr(),
            w.data_ptr(),
            n,
            ws.data_ptr(),
            ws.numel(),
            out.data_ptr(),
            _stream_handle(),
        )
        return out

    def call_ptrs(self, n: int, x_ptr: int, xs_ptr: int, ids_ptr: int, w_ptr: int, out_ptr: int,
                  stream: int, done_ptr: int = 0, done_value: int = 0) -> None:
        """The expert call on raw device pointers, enqueued on ``stream`` (a hipStream_t): bf16
        rows at x_ptr (xs_ptr = 0), or the e4m3 rows and their scales of quant_act; int32 ids and
        fp32 weights [n, k]; bf16 output [n, H]. For the serving loop, whose rows are arena
        records: no tensor is made. With ``done_ptr`` the call also answers the job
        (afd_moe_ffn_answer): the 64-bit word there becomes ``done_value`` once the output is
        visible, stored by the call's last workgroup. The caller guarantees the sizes
        (``n`` <= n_max) and the lifetimes; the C entry points check the configuration and the
        pointers."""
        if not 0 < n <= self.n_max:
            raise ValueError(f"{n} tokens outside [1, n_max={self.n_max}]")
        ws = stream_workspace(self.weights.w13.device, stream, self.layout["total"])
        if done_ptr:
            _lib.call("afd_moe_ffn_answer", ctypes.byref(self.cfg), ctypes.byref(self._wstruct),
                      None if xs_ptr else x_ptr, x_ptr if xs_ptr else None, xs_ptr or None, ids_ptr, w_ptr,
                      n, ws.data_ptr(), ws.numel(), out_ptr, done_ptr, done_value, stream)
        elif xs_ptr:
            _lib.call("afd_moe_ffn_q", ctypes.byref(self.cfg), ctypes.byref(self._wstruct), x_ptr, xs_ptr, ids_ptr,
                      w_ptr, n, ws.data_ptr(), ws.numel(), out_ptr, stream)
        else:
            _lib.call("afd_moe_ffn", ctypes.byref(self.cfg), ctypes.byref(self._wstruct), x_ptr, ids_ptr, w_ptr, n,
                      ws.data_ptr(), ws.numel(), out_ptr, stream)

    # ---- several jobs of this layer in one call ----
    def forward_batch(self, jobs, outs: Optional[list] = None) -> list:
        """One expert call over several jobs of this layer (afd_moe_ffn_batch), on the current
        stream: ``jobs`` is a list of (hidden_states, topk_output), at most AFD_MAX_BATCH of
        them and n_max tokens in all. Returns their outputs (or fills ``outs``), each equal
        bit for bit to ``forward`` on that job alone: the routing, the GEMMs and the finalize
        run once over the concatenated tokens, so each expert's weights stream once and its
        rows from different jobs share row tiles."""
        if not 1 <= len(jobs) <= _lib.AFD_MAX_BATCH:
            raise ValueError(f"a batch holds 1 to {_lib.AFD_MAX_BATCH} jobs, got {len(jobs)}")
        if outs is not None and len(outs) != len(jobs):
            raise ValueError(f"{len(jobs)} jobs but {len(outs)} outputs")
        descs = (_lib.AfdBatchJob * len(jobs))()
        keep, results, total = [], [], 0
        for b, (x, topk_output) in enumerate(jobs):
            if x.dtype != torch.bfloat16:
                raise TypeError(f"the expert path takes bf16 activations, got {x.dtype}")
            if x.dim() != 2 or x.shape[1] != self.hidden_size or not x.is_cuda:
                raise ValueError(f"x must be a device tensor [n, {self.hidden_size}], got {tuple(x.shape)} on {x.device}")
            n = x.shape[0]
            ids, w = self._topk(n, topk_output, x.device)
            x = x.contiguous()
            out = self._out(None if outs is None else outs[b], n, x.device)
            keep += [x, ids, w]
            results.append(out)
            d = descs[b]
            d.x, d.ids, d.w, d.out, d.n = x.data_ptr(), ids.data_ptr(), w.data_ptr(), out.data_ptr(), n
            total += n
        if total > self.n_max:
            raise ValueError(f"{total} tokens in the batch exceed n_max={self.n_max}")
        ws = self.workspace()
        _lib.call("afd_moe_ffn_batch", ctypes.byref(self.cfg), ctypes.byref(self._wstruct), descs, len(jobs),
                  ws.data_ptr(), ws.numel(), _stream_handle())
        return results

    def call_batch_ptrs(self, rows, stream: int, capacity: Optional[int] = None) -> None:
        """``call_ptrs`` for several jobs in one call (afd_moe_ffn_batch): ``rows`` is a list
        of (n, x_ptr, xs_ptr, ids_ptr, w_ptr, out_ptr, done_ptr, done_value), x_ptr being bf16
        rows (xs_ptr = 0) or, for every job alike, the e4m3 rows whose scales are at xs_ptr;
        each job's output goes to its out_ptr and, with done_ptr, its counter becomes
        done_value once all the batch's output is visible. ``capacity``: the most tokens a
        batch holds (default n_max), which sizes the stream's workspace."""
        capacity = self.n_max if capacity is None else capacity
        total = sum(r[0] for r in rows)
        if not 1 <= len(rows) <= _lib.AFD_MAX_BATCH or not 0 < total <= capacity:
            raise ValueError(f"{len(rows)} jobs of {total} tokens: a batch holds 1 to "
                             f"{_lib.AFD_MAX_BATCH} jobs and 1 to {capacity} tokens")
        nbytes = self._batch_bytes.get(capacity)
        if nbytes is None:
            nbytes = self._batch_bytes[capacity] = workspace_layout(self.cfg, capacity)["total"]
        ws = stream_workspace(self.weights.w13.device, stream, nbytes)
        descs = (_lib.AfdBatchJob * len(rows))()
        for d, (n, x_ptr, xs_ptr, ids_ptr, w_ptr, out_ptr, done_ptr, done_value) in zip(descs, rows):
            if xs_ptr:
                d.xq, d.xs = x_ptr, xs_ptr
            else:
                d.x = x_ptr
            d.ids, d.w, d.out, d.n = ids_ptr, w_ptr, out_ptr, n
            d.done, d.value = done_ptr or None, done_value
        _lib.call("afd_moe_ffn_batch", ctypes.byref(self.cfg), ctypes.byref(self._wstruct), descs, len(rows),
                  ws.data_ptr(), ws.numel(), stream)

    # ---- graph replay: the job is read from a device descriptor when the calls run ----
    def call_job(self, desc: torch.Tensor, n_cap: int, quantized: bool = False,
                 ws: Optional[torch.Tensor] = None) -> None:
        """Enqueue the expert call on whatever job ``desc`` (from ``new_job_desc``) holds when
        it runs, up to ``n_cap`` tokens (afd_moe_ffn_job): bf16 rows, or with ``quantized``
        the xq / xs of ``quant_act``. Capture it in a HIP graph once, then ``set_job`` +
        replay per job: no copies into static buffers, no work for tokens the job lacks.
        ``ws``: the workspace (a graph runner's own; default: the current stream's)."""
        if not 0 <= n_cap <= self.n_max:
            raise ValueError(f"n_cap {n_cap} outside [0, n_max={self.n_max}]")
        if desc.dtype != torch.uint8 or desc.numel() != JOB_BYTES or not desc.is_cuda:
            raise ValueError(f"desc must be a device uint8 tensor of {JOB_BYTES} bytes")
        if ws is None:
            ws = self.workspace()
        elif ws.dtype != torch.uint8 or ws.numel() < self.layout["total"] or not ws.is_contiguous():
            raise ValueError(f"ws must be a contiguous uint8 tensor of at least {self.layout['total']} bytes")
        _lib.call(
            "afd_moe_ffn_job",
            ctypes.byref(self.cfg),
            ctypes.byref(self._wstruct),
            desc.data_ptr(),
            n_cap,
            int(bool(quantized)),
            ws.data_ptr(),
            ws.numel(),
            _stream_handle(),
        )

    # ---- fp8 activations on the wire: A quantizes, F runs on the quantized rows ----
    @property
    def act_format(self) -> str:
        """The activation format of this layer's expert call: "mxfp8" (e4m3 + UE8M0 per 32,
        MXFP4 weights), "fp8_1x128" (e4m3 + fp32 per 128, FP8 block weights) or "bf16"."""
        if self.cfg.act_fmt == _lib.AFD_A_BF16:
            return "bf16"
        return FP8_ACT[self.weights.fmt]

    def act_scale_shape(self, n: int):
        """Shape and dtype of the activation scales of n tokens (fp8 activation formats)."""
        if self.act_format == "bf16":
            raise NotImplementedError("bf16 activations are not quantized: they have no scales")
        return act_scale_shape(self.act_format, n, self.hidden_size)

    def quant_act(self, x: torch.Tensor, q: Optional[torch.Tensor] = None, s: Optional[torch.Tensor] = None):
        """The expert call's activation quantization on its own (afd_quant_act), on the current
        stream: bf16 x [n, H] -> (q e4m3 codes uint8 [n, H], s scales)."""
        if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[1] != self.hidden_size:
            raise TypeError(f"the expert path takes bf16 [n, {self.hidden_size}] activations, got {x.dtype} {tuple(x.shape)}")
        if self.act_format == "bf16":
            raise NotImplementedError("a layer with bf16 activations does not quantize them")
        return _quant_act(self.cfg, self.act_format, x, q, s, None)

    def forward_q(self, xq: torch.Tensor, xs: torch.Tensor, topk_output, out: Optional[torch.Tensor] = None):
        """The expert call on activations quant_act (or the A side) already quantized
        (afd_moe_ffn_q); bit-identical to ``forward`` on the bf16 rows they came from."""
        n = xq.shape[0]
        shape, dtype = self.act_scale_shape(n)
        if xq.dtype != torch.uint8 or tuple(xq.shape) != (n, self.hidden_size):
            raise ValueError(f"xq must be uint8 [{n}, {self.hidden_size}], got {xq.dtype} {tuple(xq.shape)}")
        if xs.dtype != dtype or tuple(xs.shape) != shape:
            raise ValueError(f"xs must be {dtype} {shape}, got {xs.dtype} {tuple(xs.shape)}")
        if not xq.is_cuda or xs.device != xq.device:
            raise ValueError(f"xq / xs must be device tensors on one device, got {xq.device} / {xs.device}")
        ids, w = self._topk(n, topk_output, xq.device)
        out = self._out(out, n, xq.device)
        if n == 0:
            return out
        ws = self.workspace()
        _lib.call(
            "afd_moe_ffn_q",
            ctypes.byref(self.cfg),
            ctypes.byref(self._wstruct),
            xq.contiguous().data_ptr(),
            xs.contiguous().data_ptr(),
            ids.data_ptr(),
            w.data_ptr(),
            n,
            ws.data_ptr(),
            ws.numel(),
            out.data_ptr(),
            _stream_handle(),
        )
        return out

    def layout_for(self, n: int) -> dict:
        """Offsets of the workspace buffers of a call with ``n`` tokens (afd_workspace_layout)."""
        return workspace_layout(self.cfg, n)

    def ws_view(self, name: str, dtype: torch.dtype, count: int, n: int, stream=None) -> torch.Tensor:
        """A view of an intermediate buffer of the last call with ``n`` tokens (the
        workspace layout depends on n); for parity tests and profiling."""
        ws = self.workspace(stream)
        off = workspace_layout(self.cfg, n)[name]
        size = torch.tensor([], dtype=dtype).element_size()
        return ws[off : off + count * size].view(dtype)
