"""Token dispatcher of an attention (A) rank whose routed experts run on the FFN (F) ranks.

Same surface as ``python/sgl_asap_plugin/srt/layers/moe/token_dispatcher/asap.py``:
``AsapDispatcher(layer_id).dispatch(hidden_states, topk_output, micro_batch)`` enqueues the
send of one layer's tokens (empty batch -> empty output, non-standard top-k -> RuntimeError,
n > n_max -> chunked ``exchange``; :48-73) and ``combine`` returns the sum of the F ranks'
partial outputs (:75-78). ``AsapBuffer`` is the rank's connection (``send`` :149-172: bf16
check -> TypeError, int32 ids, fp32 weights, the send stream waits on the compute stream;
``recv`` :174-184: waits, then one part is cloned and several are summed in fp32, in F-rank
order, into a new bf16 tensor; ``exchange`` :186-193).

The sum is one gfx950 kernel (``afd_combine``) that can also add the shared experts' output
(``combine(..., shared_output=)``): bf16(fp32(routed) + fp32(shared)), the same two
roundings as the reference's recv followed by SGLang's plain shared add
(``srt/layers/moe/ep_moe/layer.py:29-33``).

With fp8 activations on the wire (the channel geometry's ``act``) ``send`` quantizes the
rows on the send stream first (``quant_act``, the expert call's own quantizer) and copies the
e4m3 codes and their scales: half the bytes of bf16, and the F rank skips its quantizer.

On one GPU the F rank is in-process: ``AsapBuffer.pump`` (if set) stands in for the F rank's
poll loop. It runs right after every send, so the F side enqueues a job as soon as its message
is enqueued (as a separate F process polling its doorbells would pick it up), and again before
a wait is enqueued, which keeps host order equal to causal order on the device (no stream can
ever wait on work that is enqueued after it).
"""

from __future__ import annotations

import ctypes
from typing import Callable, NamedTuple, Optional

import torch

from .. import _lib
from .experts import act_scale_shape, quant_act
from .topk import format_is_standard

# Channel slot used when the batch is not split; with two-batch overlap, micro-batch m
# travels on slot m.
SLOT = 0


class AsapDispatchOutput(NamedTuple):
    """What ``dispatch`` hands to ``combine``: either a send still waiting for its answer
    (``ticket``, with the input tensors its copies read held in ``keepalive``) or, for an empty
    or chunked batch, the finished output in ``hidden_states``."""

    ticket: Optional[object]
    hidden_states: Optional[torch.Tensor]
    keepalive: tuple = ()


def combine_parts(parts, shared: Optional[torch.Tensor], n_tokens: int, hidden: int, device) -> torch.Tensor:
    """bf16 [n, hidden] = bf16(sum_f fp32(part_f)) (+ shared) from device pointers ``parts``."""
    out = torch.empty(n_tokens, hidden, dtype=torch.bfloat16, device=device)
    if n_tokens == 0:
        return out
    arr = (ctypes.c_void_p * len(parts))(*parts)
    shared_ptr = None
    if shared is not None:
        if shared.dtype != torch.bfloat16 or tuple(shared.shape) != (n_tokens, hidden):
            raise ValueError(f"shared output must be bf16 [{n_tokens}, {hidden}], got {shared.dtype} {tuple(shared.shape)}")
        shared = shared.contiguous()
        shared_ptr = shared.data_ptr()
    _lib.call("afd_combine", arr, len(parts), shared_ptr, out.data_ptr(), n_tokens * hidden,
              torch.cuda.current_stream().cuda_stream)
    return out


class AsapDispatcher:
    def __init__(self, layer_id: int):
        self.layer_id = layer_id

    def dispatch(self, hidden_states: torch.Tensor, topk_output, micro_batch: Optional[int] = None) -> AsapDispatchOutput:
        """``micro_batch``: index of a two-batch-overlap micro-batch, None for a whole batch."""
        if hidden_states.shape[0] == 0:
            return AsapDispatchOutput(None, hidden_states.new_empty(hidden_states.shape))
        if not format_is_standard(topk_output):
            raise RuntimeError(f"ASAP sends explicit top-k ids and weights, got {type(topk_output).__name__}")
        buffer = AsapBuffer.get()
        ids, weights = topk_output.topk_ids, topk_output.topk_weights
        if hidden_states.shape[0] > buffer.n_max:
            output = buffer.exchange(self.layer_id, hidden_states, ids, weights)
            return AsapDispatchOutput(None, output)
        ticket, keepalive = buffer.send(self.layer_id, hidden_states, ids, weights, micro_batch)
        return AsapDispatchOutput(ticket, None, keepalive)

    def combine(self, combine_input: AsapDispatchOutput, shared_output: Optional[torch.Tensor] = None) -> torch.Tensor:
        if combine_input.hidden_states is not None:
            out = combine_input.hidden_states
            if shared_output is not None and out.numel():
                out = combine_parts([out.contiguous().data_ptr()], shared_output, out.shape[0], out.shape[1], out.device)
            return out
        return AsapBuffer.get().recv(combine_input.ticket, shared_output)


class AsapBuffer:
    """The attention rank's channel to the FFN ranks, with its send stream."""

    _buffer: Optional["AsapBuffer"] = None

    def __init__(self, channel, device: int, pump: Optional[Callable[[], object]] = None):
        self.channel, self.device = channel, device
        self.n_max = channel.g.n_max
        self.hidden = channel.g.hidden
        self.send_stream = torch.cuda.Stream(device)
        self._inputs_ready = torch.cuda.Event()  # recorded on the compute stream per send
        self.pump = pump
        self.act = channel.g.act
        self.stage = []
        if self.act != "bf16":
            # fp8 on the wire: one staging pair per slot; the send stream quantizes a message's
            # rows here, then copies them to the arena. The slot's next message quantizes after
            # those copies (same stream), so one pair per slot suffices.
            shape, dtype = act_scale_shape(self.act, self.n_max, self.hidden)
            self.stage = [
                (torch.empty(self.n_max, self.hidden, dtype=torch.uint8, device=device),
                 torch.empty(shape, dtype=dtype, device=device))
                for _ in range(channel.g.slots)
            ]

    @classmethod
    def get(cls) -> "AsapBuffer":
        if cls._buffer is None:
            raise RuntimeError("This attention rank is not connected to the FFN ranks")
        return cls._buffer

    @classmethod
    def install(cls, channel, device: int, pump: Optional[Callable[[], object]] = None) -> "AsapBuffer":
        cls._buffer = cls(channel, device, pump)
        return cls._buffer

    @classmethod
    def uninstall(cls) -> None:
        cls._buffer = None

    def send(self, layer_id: int, x, ids, weights, micro_batch=None):
        """Enqueue one message -> (ticket, the tensors its copies read). The send stream waits
        for the work that produced the inputs; the caller keeps them until the answer."""
        if x.dtype != torch.bfloat16:
            raise TypeError(f"ASAP carries bf16 activations, got {x.dtype}")
        given = (x, ids, weights)
        # conversions only where needed (each torch call costs host time even as a no-op)
        if not x.is_contiguous():
            x = x.contiguous()
        if ids.dtype != torch.int32 or not ids.is_contiguous():
            ids = ids.to(torch.int32).contiguous()
        if weights.dtype != torch.float32 or not weights.is_contiguous():
            weights = weights.to(torch.float32).contiguous()
        slot = SLOT if micro_batch is None else micro_batch
        n = x.shape[0]
        self._inputs_ready.record()
        self.send_stream.wait_event(self._inputs_ready)
        x_ptr, xs_ptr = x.data_ptr(), 0
        if self.stage:
            if not (0 <= slot < len(self.stage) and 1 <= n <= self.n_max):
                raise ValueError(f"slot {slot} / n_tokens {n} outside the geometry {self.channel.g}")
            q, s = self.stage[slot]
            quant_act(self.act, x, q[:n], s[:n], stream=self.send_stream)
            x_ptr, xs_ptr = q.data_ptr(), s.data_ptr()
        ticket = self.channel.send(layer_id, slot, x_ptr, ids.data_ptr(), weights.data_ptr(), n, self.send_stream,
                                   xs_ptr=xs_ptr)
        if self.pump is not None:
            self.pump()
        # The caller keeps its own tensors alive until the answer (keepalive); tensors made
        # here by a conversion are registered with the send stream, so the caching allocator
        # does not hand their memory out before the copies ran.
        for t, g in zip((x, ids, weights), given):
            if t is not g:
                t.record_stream(self.send_stream)
        return ticket, (x, ids, weights)

    def recv(self, ticket, shared: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The sum of the FFN ranks' partial outputs (plus ``shared``), as a new tensor: the
        next reply overwrites the result segments."""
        if self.pump is not None:
            self.pump()
        ptrs = self.channel.wait(ticket, torch.cuda.current_stream())
        return combine_parts(ptrs, shared, ticket.n_tokens, self.hidden, f"cuda:{self.device}")

    def exchange(self, layer_id: int, x, ids, weights) -> torch.Tensor:
        """send + recv in pieces of at most n_max tokens."""
        pieces = []
        for i in range(0, x.shape[0], self.n_max):
            end = i + self.n_max
            ticket, _ = self.send(layer_id, x[i:end], ids[i:end], weights[i:end])
            pieces.append(self.recv(ticket))
        return torch.cat(pieces)
