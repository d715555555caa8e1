"""GPU: the largest shapes the expert call accepts, against the fp32 CPU oracle.

* hidden at its limit (16384) with 64 local experts whose packed gate/up weights span more
  than 4 GiB (MXFP4 4.6 GB, FP8-block 8.6 GB) and down weights more than 2 GiB, so the GEMMs
  take expert offsets past 2^32 bytes; the tokens go to the first, middle and last experts,
  and some only to experts of another rank. The 64 experts repeat a pool of three distinct
  ones (expert e holds pool member e % 3), so the oracle needs only the pool's weights; an
  offset that wrapped at 2^32 would read the middle of another expert's image.
* the intermediate size at its limit (16384) with a small hidden size.
* the largest job (131071 tokens) at hidden 16384: token rows at 32-bit byte offsets up to
  2^31 (fp8 rows) and 2^32 (bf16 rows) minus a row.

Both weight formats, with fp8 and with bf16 activations; the bars of the other layer tests
(rel-L2 <= 1e-2, tokens with no local expert exactly zero). The weights are drawn so that
each format holds them exactly (every block: codes times a power-of-two scale, with one
element at the format's largest code, so the quantizer picks that scale and rounds
nothing): the oracle's dequantized weights are then the drawn values themselves (checked on
the CPU below), instead of a CPU quantization of a billion values; they are drawn on the GPU.
"""

import numpy as np
import pytest
import torch

from gpu_util import dev, say
from oracle import experts as OX
from oracle import formats as F
from sgl_asap_amd import workloads as W
from sgl_asap_amd.moe.experts import AfdExperts, ExpertWeights, pack_fp8_block_experts, pack_mxfp4_experts
from sgl_asap_amd.moe.topk import StandardTopKOutput
from test_gpu_moe import assert_close

HIDDEN, INTER = 16384, 4096
NUM_LOCAL, NUM_EXPERTS, POOL = 64, 66, 3
USED = (0, 1, 31, 32, 62, 63)  # local experts the tokens go to
N_TOKENS = 48

_E4M3_CODES = np.array([c for c in range(256) if c & 0x7F != 0x7F], dtype=np.uint8)


def exact_matrix(fmt, rows, cols, gen, device):
    """fp32 [rows, cols] that the weight format holds exactly. MXFP4 (blocks of 32 along a
    row): e2m1 values times 2^k, element 0 of each block +-6 (the largest e2m1 value), so the
    block exponent is k. FP8-block (128 x 128 blocks): e4m3 values times 2^k, one element
    +-448, so the block scale max|v| / 448 is 2^k. k is drawn per block, the magnitudes
    near 0.02 rms."""
    def draw(hi, shape):
        return torch.randint(0, hi, shape, generator=gen, device=device)

    sign = lambda shape, m: torch.where(draw(2, shape) == 1, m, -m)
    if fmt == "mxfp4":
        vals = torch.from_numpy(np.concatenate([F.E2M1_VALUES, -F.E2M1_VALUES]).astype(np.float32)).to(device)
        v = vals[draw(16, (rows, cols // 32, 32))]
        v[:, :, 0] = sign((rows, cols // 32), 6.0)
        k = draw(2, (rows, cols // 32, 1)) - 8
    else:
        vals = torch.from_numpy(F.e4m3_decode(_E4M3_CODES).astype(np.float32)).to(device)
        v = vals[draw(len(_E4M3_CODES), (rows // 128, 128, cols // 128, 128))]
        v[:, 0, :, 0] = sign((rows // 128, cols // 128), 448.0)
        k = draw(2, (rows // 128, 1, cols // 128, 1)) - 13
    return (v * torch.exp2(k.to(torch.float32))).reshape(rows, cols)


def exact_weights(fmt, num, hidden, inter, seed, device):
    """Logical w13 [num, 2I, H] and w2 [num, H, I] (fp32 tensors on ``device``) the format
    holds exactly."""
    gen = W.generator(device, seed)
    w13 = torch.stack([exact_matrix(fmt, 2 * inter, hidden, gen, device) for _ in range(num)])
    w2 = torch.stack([exact_matrix(fmt, hidden, inter, gen, device) for _ in range(num)])
    return w13, w2


@pytest.mark.parametrize("fmt", ["mxfp4", "fp8_block"])
def test_exact_weights_survive_the_oracle_quantizer(fmt):
    """CPU: the oracle's weight quantizer returns the drawn weights bit for bit."""
    w13, w2 = (t.numpy() for t in exact_weights(fmt, 1, 512, 256, seed=3, device="cpu"))
    for w in (w13, w2):
        if fmt == "mxfp4":
            deq = F.mx_dequantize(*F.mx_quantize(w, "e2m1"), "e2m1")
        else:
            deq = F.fp8_block_dequantize_2d(*F.fp8_block_quantize_2d(w))
        assert np.array_equal(deq.view(np.uint32), w.view(np.uint32))
    assert 0.01 < float(np.sqrt(np.mean(np.square(w13)))) < 0.04


def packed(fmt, w13, w2):
    pack = pack_mxfp4_experts if fmt == "mxfp4" else pack_fp8_block_experts
    return pack(w13, w2, device=dev())


class PoolView:
    """[NUM_LOCAL, ...] weights as the oracle indexes them: expert e is pool member e % POOL."""

    def __init__(self, arrays):
        self.arrays = arrays
        self.shape = (NUM_LOCAL,) + arrays.shape[1:]

    def __getitem__(self, e):
        return self.arrays[e % POOL]


def grown(pool: ExpertWeights) -> ExpertWeights:
    """The pool's packed experts repeated to NUM_LOCAL experts (expert e = member e % POOL)."""

    def grow(t):
        if t.numel() == 0:
            return t
        out = torch.empty((NUM_LOCAL,) + tuple(t.shape[1:]), dtype=t.dtype, device=t.device)
        for e in range(NUM_LOCAL):
            out[e].copy_(t[e % POOL])
        return out

    return ExpertWeights(pool.fmt, NUM_LOCAL, pool.hidden, pool.inter, grow(pool.w13), grow(pool.s13),
                         grow(pool.w2), grow(pool.s2))


def routing():
    """Token t goes to two distinct experts of USED, or (every eighth token) to the two
    experts past the local range; weights positive, summing to 1."""
    rng = np.random.default_rng(5)
    ids = np.empty((N_TOKENS, 2), dtype=np.int32)
    for t in range(N_TOKENS):
        if t % 8 == 7:
            ids[t] = (NUM_LOCAL, NUM_LOCAL + 1)
        else:
            a = t % len(USED)
            ids[t] = (USED[a], USED[(a + 1 + (t // len(USED)) % (len(USED) - 1)) % len(USED)])
    w = rng.uniform(0.1, 1.0, (N_TOKENS, 2)).astype(np.float32)
    return ids, w / w.sum(axis=1, keepdims=True)


def oracle_act(fmt, act_format):
    return "bf16" if act_format == "bf16" else "mxfp8" if fmt == "mxfp4" else "fp8_1x128"


@pytest.mark.gpu
@pytest.mark.parametrize("act_format", [None, "bf16"])
@pytest.mark.parametrize("fmt", ["mxfp4", "fp8_block"])
def test_weights_past_4gib(fmt, act_format):
    say(f"large fmt={fmt} act_format={act_format} H={HIDDEN} I={INTER} local={NUM_LOCAL} used={USED}")
    w13, w2 = exact_weights(fmt, POOL, HIDDEN, INTER, seed=77, device=dev())
    weights = grown(packed(fmt, w13, w2))
    w13, w2 = w13.cpu().numpy(), w2.cpu().numpy()
    assert weights.w13.numel() > 2**32 and weights.w2.numel() > 2**31
    x = W.tokens(N_TOKENS, HIDDEN, W.generator("cpu", 78), "cpu")
    ids, w = routing()
    experts = AfdExperts(NUM_EXPERTS, 2, 0, range(NUM_LOCAL), weights, n_max=N_TOKENS, act_format=act_format)
    out = experts(x.to(dev()), StandardTopKOutput(torch.from_numpy(w).to(dev()), torch.from_numpy(ids).to(dev())))
    torch.cuda.synchronize()
    del experts, weights
    ref = OX.moe_ffn(x, ids, w, PoolView(w13), PoolView(w2), 0, act=oracle_act(fmt, act_format))
    assert_close(out, ref, ids, range(NUM_LOCAL))


@pytest.mark.gpu
@pytest.mark.parametrize("act_format", [None, "bf16"])
@pytest.mark.parametrize("fmt", ["mxfp4", "fp8_block"])
def test_largest_inter(fmt, act_format):
    hidden, inter, n = 1024, 16384, 100
    say(f"largest inter fmt={fmt} act_format={act_format} H={hidden} I={inter} local=[1, 3) of 4, n={n}")
    w13, w2 = exact_weights(fmt, 2, hidden, inter, seed=79, device=dev())
    gen = W.generator("cpu", 80)
    x = W.tokens(n, hidden, gen, "cpu")
    ids, w = W.route_uniform(n, 4, 2, gen, "cpu")
    experts = AfdExperts(4, 2, 0, range(1, 3), packed(fmt, w13, w2), n_max=n, act_format=act_format)
    out = experts(x.to(dev()), StandardTopKOutput(w.to(dev()), ids.to(dev())))
    torch.cuda.synchronize()
    ref = OX.moe_ffn(x, ids.numpy(), w.numpy(), w13.cpu().numpy(), w2.cpu().numpy(), 1,
                     act=oracle_act(fmt, act_format))
    assert_close(out, ref, ids.numpy(), range(1, 3))


@pytest.mark.gpu
@pytest.mark.parametrize("act_format", [None, "bf16"])
@pytest.mark.parametrize("fmt", ["mxfp4", "fp8_block"])
def test_largest_job_at_the_hidden_limit(fmt, act_format):
    """131071 tokens (the most a call takes) of hidden 16384: token rows at byte offsets up
    to 2^31 (fp8 rows) and 2^32 (bf16 rows) minus a row. The first and last 1000 tokens, run
    as a job of their own, give the same rows bit for bit, and the last 64 match the oracle."""
    hidden, inter, num, k, n = HIDDEN, 128, 8, 2, 131071
    say(f"largest job fmt={fmt} act_format={act_format} H={hidden} I={inter} E={num} k={k} n={n}")
    w13, w2 = exact_weights(fmt, num, hidden, inter, seed=83, device=dev())
    gen = W.generator(dev(), 84)
    x = W.tokens(n, hidden, gen, dev())
    ids, w = W.route_uniform(n, num, k, gen, dev())
    experts = AfdExperts(num, k, 0, range(num), packed(fmt, w13, w2), n_max=n, act_format=act_format)
    out = experts(x, StandardTopKOutput(w, ids))
    ends = torch.cat([torch.arange(1000), torch.arange(n - 1000, n)]).to(dev())
    sub = experts(x[ends].contiguous(), StandardTopKOutput(w[ends].contiguous(), ids[ends].contiguous()))
    torch.cuda.synchronize()
    assert torch.equal(sub.view(torch.int16), out[ends].view(torch.int16))
    last = slice(n - 64, n)
    xl, idl, wl = x[last].cpu(), ids[last].cpu().numpy(), w[last].cpu().numpy()
    got = out[last]
    del experts, out, sub, x
    ref = OX.moe_ffn(xl, idl, wl, w13.cpu().numpy(), w2.cpu().numpy(), 0, act=oracle_act(fmt, act_format))
    assert_close(got, ref, idl, range(num))
