"""Arena layout, doorbell word and error types shared by the A side and the F side.

Restates the wire contract of ``python/sgl_asap_plugin/transport/layout.py`` (the whole
file): the same region offsets, alignment, doorbell bit fields, range checks and
exception classes, so a Geometry computed here and one computed by the reference agree
field by field.

One message is one micro-batch (slot ``s``) of one MoE layer from A rank ``a``. On one
MI355X both ends live on the same device:

    producer (A) stream                      consumer (F) stream
      wait   done(f, s) == seq - 1             wait   bell(a, s) == seq
      copy   x, ids, w -> recv region(a, s)    experts(x, ids, w) -> seg(f, s)
      write  bell(a, s) := doorbell word       write  done(f, s) := seq
    compute stream: shared experts, wait done(f, s) == seq, combine

RecvArena (device memory, F owns), one region per (a, s):
    | x [n_max, hidden] bf16 | ids [n_max, topk] i32 | w [n_max, topk] f32 |
    0                      ids_off                 w_off            region_bytes

With ``act`` = "mxfp8" or "fp8_1x128" (fp8 activations on the wire, the reference's TODO at
scripts/run_asap.sh:110-111) A quantizes before the copy and the x field becomes
    | xq [n_max, hidden] e4m3 | xs [n_max, scale_bytes/token] | ids ... | w ... |
    0                        xs_off                          ids_off
where a token's scales are hidden/32 UE8M0 bytes ("mxfp8", the MXFP4 experts' input) or
hidden/128 fp32 ("fp8_1x128", the FP8 block experts' input). Results stay bf16.

Flags (doorbells of F, done flags of A): one 64-byte line per flag. This build keeps
them in pinned host memory so a host thread can always release a parked stream wait
with a plain store; the offsets are the reference's.

ResultArena (device memory, A owns):
    | done flags page (FLAGS_PAGE) | seg(f=0, s=0) [n_max, hidden] bf16 | seg(0, 1) | ...

Doorbell bits: 0-31 seq | 32-48 n_tokens (1..MAX_TOKENS) | 49-58 layer (0..MAX_LAYER) |
59-63 epoch (1..MAX_EPOCH).
"""

from __future__ import annotations

from dataclasses import asdict, dataclass, fields

ALIGN = 256
FLAG_STRIDE = 64
FLAGS_PAGE = 2 << 20
BELL_STRIDE = 64
ACT_BYTES = 2  # bf16 activations on the wire
ACT_FORMATS = ("bf16", "mxfp8", "fp8_1x128")
ID_BYTES = 4  # int32 global expert ids
W_BYTES = 4  # fp32 top-k weights

PROTO_VERSION = 4
PROTO_VERSION_FP8_WIRE = 5  # the x field carries e4m3 codes + scales (Geometry.act != "bf16")
SEQ_MASK = 0xFFFFFFFF
MAX_TOKENS = (1 << 17) - 1
MAX_LAYER = (1 << 10) - 1
MAX_EPOCH = (1 << 5) - 1

_N_SHIFT, _LAYER_SHIFT, _EPOCH_SHIFT = 32, 49, 59


class TransportError(RuntimeError):
    """Any failure of the A<->F transport (layout.py:75-76 of the reference)."""


class HandshakeError(TransportError):
    """The peer could not be reached or refused the connection (layout.py:79-80)."""


class ChannelPoisoned(TransportError):
    """A stream wait timed out and was released by the watchdog; every result still in
    flight is garbage until ``reconnect()`` (layout.py:83-84)."""


def align_up(n: int, a: int = ALIGN) -> int:
    """Smallest multiple of ``a`` that is >= ``n`` (layout.py:87-89)."""
    return (n + a - 1) // a * a


def pack_doorbell(seq: int, n_tokens: int, layer_id: int, epoch: int) -> int:
    """64-bit doorbell word; out-of-range n_tokens / layer / epoch raise ValueError.

    Follows layout.py:92-102: seq is taken modulo 2^32, the other fields are checked.
    """
    ok = 1 <= n_tokens <= MAX_TOKENS and 0 <= layer_id <= MAX_LAYER and 1 <= epoch <= MAX_EPOCH
    if not ok:
        raise ValueError(
            f"doorbell field out of range: n_tokens={n_tokens} layer_id={layer_id} epoch={epoch}"
        )
    return (
        (seq & SEQ_MASK)
        | (n_tokens << _N_SHIFT)
        | (layer_id << _LAYER_SHIFT)
        | (epoch << _EPOCH_SHIFT)
    )


def unpack_doorbell(word: int):
    """-> (seq, n_tokens, layer_id, epoch), the inverse of pack_doorbell (layout.py:105-113)."""
    return (
        word & SEQ_MASK,
        (word >> _N_SHIFT) & MAX_TOKENS,
        (word >> _LAYER_SHIFT) & MAX_LAYER,
        (word >> _EPOCH_SHIFT) & MAX_EPOCH,
    )


def seq_ahead(new: int, last: int) -> int:
    """Cyclic int32 difference new - last, the wrap-safe ordering of sequence numbers
    (server.py:266-268 compares doorbell seqs this way)."""
    d = (new - last) & SEQ_MASK
    return d - (1 << 32) if d >= 1 << 31 else d


@dataclass(frozen=True)
class Geometry:
    """Sizes of one deployment (layout.py:116-198). Every field but ``act`` is a positive
    int; ``act`` is the activation format on the wire (one of ACT_FORMATS, default bf16,
    which keeps the reference's layout byte for byte)."""

    num_a: int  # A ranks (replicas x group)
    group: int  # A ranks of one replica; their rows form one F job
    slots: int  # micro-batches in flight per A rank
    n_max: int  # tokens per message, at most MAX_TOKENS
    hidden: int
    topk: int
    num_f: int  # F ranks
    act: str = "bf16"

    def __post_init__(self):
        bad = []
        for f in fields(self):
            if f.name == "act":
                continue
            v = getattr(self, f.name)
            if not isinstance(v, int) or isinstance(v, bool) or v < 1:
                bad.append(f"{f.name}={v!r}")
        if self.act not in ACT_FORMATS:
            bad.append(f"act={self.act!r} is not one of {ACT_FORMATS}")
        if not bad and self.num_a % self.group:
            bad.append(f"num_a={self.num_a} is not a multiple of group={self.group}")
        if not bad and self.n_max > MAX_TOKENS:
            bad.append(f"n_max={self.n_max} exceeds the {MAX_TOKENS} tokens a doorbell can announce")
        if not bad and self.act != "bf16" and self.hidden % 128:
            bad.append(f"act={self.act} needs hidden={self.hidden} to be a multiple of 128")
        if bad:
            raise ValueError("invalid transport geometry: " + ", ".join(bad))

    @property
    def proto_version(self) -> int:
        """The wire protocol of this geometry: the reference's for bf16 activations, the next
        one when fp8 activations change the x field."""
        return PROTO_VERSION if self.act == "bf16" else PROTO_VERSION_FP8_WIRE

    # activations on the wire
    @property
    def x_bytes_per_token(self) -> int:
        """Bytes of one token's codes in the x field (bf16: 2 per element, fp8: 1)."""
        return self.hidden * (ACT_BYTES if self.act == "bf16" else 1)

    @property
    def xs_bytes_per_token(self) -> int:
        """Bytes of one token's activation scales (0 for bf16)."""
        if self.act == "mxfp8":
            return self.hidden // 32
        if self.act == "fp8_1x128":
            return self.hidden // 128 * 4
        return 0

    # RecvArena of an F rank
    @property
    def xs_off(self) -> int:
        return align_up(self.n_max * self.x_bytes_per_token)

    @property
    def ids_off(self) -> int:
        return self.xs_off + align_up(self.n_max * self.xs_bytes_per_token)

    @property
    def w_off(self) -> int:
        return self.ids_off + align_up(self.n_max * self.topk * ID_BYTES)

    @property
    def region_bytes(self) -> int:
        return self.w_off + align_up(self.n_max * self.topk * W_BYTES)

    @property
    def recv_bytes(self) -> int:
        return self.num_a * self.slots * self.region_bytes

    def region_off(self, a: int, s: int) -> int:
        return (a * self.slots + s) * self.region_bytes

    # doorbell page of an F rank
    @property
    def host_bytes(self) -> int:
        return align_up(self.num_a * self.slots * BELL_STRIDE, 4096)

    def bell_off(self, a: int, s: int) -> int:
        return (a * self.slots + s) * BELL_STRIDE

    # ResultArena of an A rank
    @property
    def flags_bytes(self) -> int:
        return align_up(self.num_f * self.slots * FLAG_STRIDE, FLAGS_PAGE)

    @property
    def seg_bytes(self) -> int:
        return align_up(self.n_max * self.hidden * ACT_BYTES)

    @property
    def result_bytes(self) -> int:
        return self.flags_bytes + self.num_f * self.slots * self.seg_bytes

    def done_off(self, f: int, s: int) -> int:
        return (f * self.slots + s) * FLAG_STRIDE

    def seg_off(self, f: int, s: int) -> int:
        return self.flags_bytes + (f * self.slots + s) * self.seg_bytes

    def as_dict(self) -> dict:
        return asdict(self)

    @classmethod
    def from_dict(cls, d: dict) -> "Geometry":
        return cls(**{f.name: d[f.name] for f in fields(cls) if f.name in d or f.name != "act"})
