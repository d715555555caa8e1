"""GPU: the one-GPU AFD loop (dispatch -> arena copies + doorbell -> F job gated on the
doorbell -> reply + done flag -> combine) returns exactly what the expert call returns."""

import numpy as np
import pytest
import torch

from gpu_util import bits16, dev, say
from oracle import experts as OX
from sgl_asap_amd import workloads as W
from sgl_asap_amd.loop import OneGpuAfd
from sgl_asap_amd.moe.experts import AfdExperts, pack_mxfp4_experts
from sgl_asap_amd.moe.layer import AsapMoE
from sgl_asap_amd.moe.topk import StandardTopKOutput

pytestmark = pytest.mark.gpu

H, I, E, K = 256, 128, 16, 4
LOCAL = range(0, 8)  # this F rank owns half the experts


def make_experts(n_max, layers=(0,), seed=0):
    gen = W.generator("cpu", seed)
    out = {}
    for layer in layers:
        w13, w2 = W.expert_weights(len(LOCAL), H, I, gen, "cpu")
        out[layer] = AfdExperts(E, K, layer, LOCAL, pack_mxfp4_experts(w13, w2, device=dev()), n_max=n_max)
    return out


def job(n, seed):
    gen = W.generator("cpu", seed)
    x = W.tokens(n, H, gen, "cpu").to(dev())
    ids, w = W.route_uniform(n, E, K, gen, "cpu")
    return x, StandardTopKOutput(w.to(dev()), ids.to(dev()))


def direct(experts, layer, x, topk):
    out = experts[layer](x, topk)
    torch.cuda.synchronize()
    return bits16(out)


def test_loop_matches_expert_call():
    say("loop: single layer, single slot")
    experts = make_experts(64)
    with OneGpuAfd(experts, n_max=64) as afd:
        layer = AsapMoE(E, H, I, 0, top_k=K)
        for seed in range(3):
            x, topk = job(37 + seed, seed)
            out = layer(x, topk)
            torch.cuda.synchronize()
            assert np.array_equal(bits16(out), direct(experts, 0, x, topk))
        assert afd.server.stats["jobs"] == 3 and afd.server.stats["lost_messages"] == 0


def test_loop_shared_expert_add():
    say("loop: shared expert added in the combine")
    experts = make_experts(64)
    gen = W.generator("cpu", 5)
    wsh = torch.randn(H, H, generator=gen).to(torch.bfloat16).to(dev()) * 0.05

    def shared(x):
        return (x.float() @ wsh.float().T).to(torch.bfloat16)

    with OneGpuAfd(experts, n_max=64):
        layer = AsapMoE(E, H, I, 0, top_k=K, shared_experts=shared)
        x, topk = job(50, 11)
        out = layer(x, topk)
        torch.cuda.synchronize()
        routed = direct(experts, 0, x, topk)
        ref = OX.combine([routed], bits16(shared(x)))
        assert np.array_equal(bits16(out), ref)


def test_two_micro_batches_in_flight():
    say("loop: two slots in flight")
    experts = make_experts(64, layers=(0, 1))
    with OneGpuAfd(experts, n_max=64, slots=2):
        layers = [AsapMoE(E, H, I, lid, top_k=K) for lid in (0, 1)]
        for lid, layer in enumerate(layers):
            (xa, ta), (xb, tb) = job(20, 2 * lid), job(33, 2 * lid + 1)
            da = layer.dispatcher.dispatch(xa, ta, micro_batch=0)
            db = layer.dispatcher.dispatch(xb, tb, micro_batch=1)
            oa = layer.dispatcher.combine(da)
            ob = layer.dispatcher.combine(db)
            torch.cuda.synchronize()
            assert np.array_equal(bits16(oa), direct(experts, lid, xa, ta))
            assert np.array_equal(bits16(ob), direct(experts, lid, xb, tb))


def test_chained_layers_without_synchronization():
    """Consecutive layers as a serving loop runs them: each micro-batch's next send reads the
    combine output of its previous layer (made on the compute stream, still in flight), the
    slots are reused every layer, and nothing synchronizes until the end. Every layer's output
    equals the expert call on the previous output, bit for bit."""
    say("loop: 4 chained layers x 2 micro-batches, no host synchronization")
    experts = make_experts(64, layers=(0, 1))
    with OneGpuAfd(experts, n_max=64, slots=2) as afd:
        layers = [AsapMoE(E, H, I, lid, top_k=K) for lid in (0, 1)]
        starts = [job(40, 500), job(29, 501)]
        xs = [x for x, _ in starts]
        outs = []
        for step in range(4):
            layer = layers[step % 2]
            d = [layer.dispatcher.dispatch(xs[m], starts[m][1], micro_batch=m) for m in range(2)]
            xs = [layer.dispatcher.combine(d[m]) for m in range(2)]
            outs.append(list(xs))
        torch.cuda.synchronize()
        ref = [x for x, _ in starts]
        for step in range(4):
            ref = [experts[step % 2](ref[m], starts[m][1]) for m in range(2)]
            torch.cuda.synchronize()
            for m in range(2):
                assert np.array_equal(bits16(outs[step][m]), bits16(ref[m])), (step, m)
        assert afd.server.stats["jobs"] == 8 and afd.server.stats["lost_messages"] == 0


def test_sequence_wrap():
    say("loop: seq_base 2^32 - 3, eight messages across the wrap")
    experts = make_experts(64)
    with OneGpuAfd(experts, n_max=64, slots=1, seq_base=(1 << 32) - 3) as afd:
        layer = AsapMoE(E, H, I, 0, top_k=K)
        for seed in range(8):
            x, topk = job(16 + seed, 100 + seed)
            out = layer(x, topk)
            torch.cuda.synchronize()
            assert np.array_equal(bits16(out), direct(experts, 0, x, topk))
        # the doorbells' 32-bit sequence field wrapped after 2 messages; the done counter did not
        assert afd.channel.done_count(0, 0) == (1 << 32) - 3 + 8
        assert afd.server.stats["jobs"] == 8 and afd.server.stats["lost_messages"] == 0


def test_exchange_above_n_max():
    say("loop: n > n_max is exchanged in pieces")
    experts = make_experts(128)
    with OneGpuAfd(experts, n_max=48):
        layer = AsapMoE(E, H, I, 0, top_k=K)
        x, topk = job(128, 7)
        out = layer(x, topk)
        torch.cuda.synchronize()
        assert np.array_equal(bits16(out), direct(experts, 0, x, topk))


def test_graph_buckets():
    say("loop: hip graph buckets up to 64 tokens")
    experts = make_experts(64)
    with OneGpuAfd(experts, n_max=64, graph_max_tokens=64) as afd:
        assert afd.scheduler.graph_runner.buckets == [1, 2, 4, 8, 16, 32, 64]
        layer = AsapMoE(E, H, I, 0, top_k=K)
        for n in (1, 3, 16, 17, 64):
            x, topk = job(n, 200 + n)
            out = layer(x, topk)
            torch.cuda.synchronize()
            assert np.array_equal(bits16(out), direct(experts, 0, x, topk)), n


def test_empty_batch():
    say("loop: empty batch")
    experts = make_experts(64)
    with OneGpuAfd(experts, n_max=64) as afd:
        layer = AsapMoE(E, H, I, 0, top_k=K)
        x, topk = job(0, 1)
        out = layer(x, topk)
        assert out.shape == (0, H) and afd.server.stats["jobs"] == 0


def test_two_replicas_two_slots():
    say("loop: 2 A replicas x 2 slots into one F server, 3 rounds")
    experts = make_experts(64)
    with OneGpuAfd(experts, n_max=64, slots=2, replicas=2) as afd:
        sends = [torch.cuda.Stream() for _ in range(2)]
        main = torch.cuda.current_stream()
        for rnd in range(3):
            jobs, tickets = [], []
            for r in range(2):
                for mb in range(2):
                    x, topk = job(10 + 7 * r + 3 * mb + rnd, 300 + 10 * rnd + 2 * r + mb)
                    ids = topk.topk_ids.to(torch.int32).contiguous()
                    w = topk.topk_weights.to(torch.float32).contiguous()
                    sends[r].wait_stream(main)
                    t = afd.channels[r].send(0, mb, x.data_ptr(), ids.data_ptr(), w.data_ptr(), x.shape[0], sends[r])
                    jobs.append((r, x, topk, ids, w))
                    tickets.append((r, t))
            assert afd.scheduler.serve_pending() == 4
            for (r, t), (_, x, topk, _, _) in zip(tickets, jobs):
                ptr = afd.channels[r].wait(t, main)[0]
                got = torch.empty(x.shape[0], H, dtype=torch.bfloat16, device=dev())
                _lib_copy(got, ptr)
                torch.cuda.synchronize()
                assert np.array_equal(bits16(got), direct(experts, 0, x, topk)), (rnd, r)
        assert afd.server.stats["jobs"] == 12 and afd.server.stats["lost_messages"] == 0


def _lib_copy(dst, src_ptr):
    from sgl_asap_amd.transport import hip

    hip.copy_async(dst.data_ptr(), src_ptr, dst.numel() * 2, torch.cuda.current_stream().cuda_stream)


def test_graph_replays_match_eager_every_time():
    """Each captured bucket graph replayed several times, with eager expert calls and
    synchronizations between the replays: every replay equals the eager result bit for bit."""
    from sgl_asap_amd.runner.graph_runner import FfnGraphRunner

    say("graphs: repeated replays interleaved with eager calls")
    experts = make_experts(64)
    runner = FfnGraphRunner(experts, 64, LOCAL)
    for rep in range(4):
        for n in (5, 16, 33):
            x, topk = job(n, 500 + 10 * rep + n)
            ids = topk.topk_ids.to(torch.int32)
            got = runner.run(0, x, ids, topk.topk_weights, buffer=rep % 2)
            torch.cuda.synchronize()
            got_bits = bits16(got)
            want = direct(experts, 0, x, topk)  # eager work between the replays
            assert np.array_equal(got_bits, want), (rep, n)


@pytest.mark.parametrize("graphs", [0, 64])
def test_group_of_two_a_ranks(graphs):
    """Two A ranks of one replica (a TP group): their rows form one F job, concatenated row
    by row; each rank's answer equals the expert call on its own rows (eager and graphs)."""
    say(f"loop: a group of 2 A ranks, bf16, graph_max_tokens={graphs}")
    experts = make_experts(64)
    with OneGpuAfd(experts, n_max=64, group=2, graph_max_tokens=graphs) as afd:
        sends = [torch.cuda.Stream() for _ in range(2)]
        main = torch.cuda.current_stream()
        for rnd in range(2):
            keep, tickets = [], []
            for r in range(2):
                x, topk = job(13 + 17 * r + rnd, 700 + 10 * rnd + r)
                ids = topk.topk_ids.to(torch.int32).contiguous()
                w = topk.topk_weights.to(torch.float32).contiguous()
                sends[r].wait_stream(main)
                tickets.append(afd.channels[r].send(0, 0, x.data_ptr(), ids.data_ptr(), w.data_ptr(), x.shape[0],
                                                    sends[r]))
                keep.append((x, topk, ids, w))
            assert afd.scheduler.serve_pending() == 1
            for r, (t, (x, topk, _, _)) in enumerate(zip(tickets, keep)):
                ptr = afd.channels[r].wait(t, main)[0]
                got = torch.empty(x.shape[0], H, dtype=torch.bfloat16, device=dev())
                _lib_copy(got, ptr)
                torch.cuda.synchronize()
                assert np.array_equal(bits16(got), direct(experts, 0, x, topk)), (rnd, r)
        assert afd.server.stats["jobs"] == 2


def _send(afd, r, slot, x, topk, stream):
    ids = topk.topk_ids.to(torch.int32).contiguous()
    w = topk.topk_weights.to(torch.float32).contiguous()
    stream.wait_stream(torch.cuda.current_stream())
    t = afd.channels[r].send(0, slot, x.data_ptr(), ids.data_ptr(), w.data_ptr(), x.shape[0], stream)
    return t, (x, ids, w)


def test_group_jobs_served_back_to_back():
    """A group of 2 A ranks, eager: two jobs served one after the other with no host
    synchronization between them; each job's output buffer is only reused after its reply
    copies ran, so both answers are right."""
    say("loop: group of 2, two eager jobs back to back")
    experts = make_experts(64)
    with OneGpuAfd(experts, n_max=64, slots=2, group=2) as afd:
        sends = [torch.cuda.Stream() for _ in range(2)]
        main = torch.cuda.current_stream()
        keep, tickets = [], []
        for slot in range(2):
            for r in range(2):
                x, topk = job(9 + 11 * r + 5 * slot, 800 + 2 * slot + r)
                t, held = _send(afd, r, slot, x, topk, sends[r])
                tickets.append((r, t))
                keep.append((x, topk, held))
        assert afd.scheduler.serve_pending() == 2
        got = []
        for r, t in tickets:
            afd.channels[r].wait(t, main)
            got.append(afd.channels[r].result_view(0, t.slot, t.n_tokens).clone())
        torch.cuda.synchronize()
        for (x, topk, _), g in zip(keep, got):
            assert np.array_equal(bits16(g), direct(experts, 0, x, topk))


def test_two_sends_on_one_slot_before_serving():
    """The producer posts message 2 of a slot before anything served message 1: its stream
    must wait for the answer to 1 before overwriting the region, so the send first serves
    what is pending (message 1's job is enqueued before that wait, whatever hardware queues
    the streams share), then F serves 2, and the answer to 2 is right."""
    say("loop: two sends on one slot before a poll")
    experts = make_experts(64)
    with OneGpuAfd(experts, n_max=64, slots=1) as afd:
        send = torch.cuda.Stream()
        main = torch.cuda.current_stream()
        (x1, k1), (x2, k2) = job(21, 901), job(30, 902)
        t1, h1 = _send(afd, 0, 0, x1, k1, send)
        t2, h2 = _send(afd, 0, 0, x2, k2, send)
        assert (t1.seq, t2.seq) == (1, 2)
        assert afd.server.stats["jobs"] == 1  # message 1, served by the second send
        assert afd.scheduler.serve_pending() == 1
        assert afd.server.stats["jobs"] == 2
        afd.channel.wait(t2, main)
        got = afd.channel.result_view(0, 0, t2.n_tokens).clone()
        torch.cuda.synchronize()
        assert np.array_equal(bits16(got), direct(experts, 0, x2, k2))
        assert afd.server.stats["lost_messages"] == 0 and afd.channel.done_count(0, 0) == 2


def test_group_of_two_two_sends_per_slot():
    """A group of 2 A ranks on one slot, two messages each. Rank 0's first row is taken by a
    poll and waits in a half-formed job; a second send of rank 0 before rank 1's first message
    is refused (no job could answer its backpressure wait yet) with nothing enqueued. Once rank
    1's first word is in the inbox, rank 0's second send serves the completed job before its
    stream waits for the answer, so the wait never sits ahead of its job on a shared hardware
    queue; the answers to the second messages are right."""
    say("loop: group of 2, two sends per slot")
    experts = make_experts(64)
    with OneGpuAfd(experts, n_max=64, slots=1, group=2) as afd:
        sends = [torch.cuda.Stream() for _ in range(2)]
        main = torch.cuda.current_stream()
        msgs = [[job(11 + 3 * r + 7 * m, 950 + 10 * m + r) for r in range(2)] for m in range(2)]
        held = []
        _, h = _send(afd, 0, 0, *msgs[0][0], sends[0])
        held.append(h)
        assert afd.scheduler.serve_pending() == 0  # rank 0's row taken: half a job
        with pytest.raises(RuntimeError, match="other A"):
            _send(afd, 0, 0, *msgs[1][0], sends[0])
        assert afd.channels[0]._count[0] == 1  # the refused send took no sequence number
        _, h = _send(afd, 1, 0, *msgs[0][1], sends[1])  # its word waits in the inbox
        held.append(h)
        assert afd.server.stats["jobs"] == 0
        t0, h = _send(afd, 0, 0, *msgs[1][0], sends[0])  # serves job 1 before its wait
        held.append(h)
        assert afd.server.stats["jobs"] == 1 and t0.seq == 2
        t1, h = _send(afd, 1, 0, *msgs[1][1], sends[1])
        held.append(h)
        assert afd.scheduler.serve_pending() == 1
        got = []
        for r, t in ((0, t0), (1, t1)):
            afd.channels[r].wait(t, main)
            got.append(afd.channels[r].result_view(0, 0, t.n_tokens).clone())
        torch.cuda.synchronize()
        for r in range(2):
            assert np.array_equal(bits16(got[r]), direct(experts, 0, *msgs[1][r])), r
            assert afd.channels[r].done_count(0, 0) == 2
        assert afd.server.stats["jobs"] == 2 and afd.server.stats["lost_messages"] == 0


def test_stall_releases_the_parked_wait_and_poisons():
    """A message whose doorbell carries a wrong epoch is dropped by the F server, so its reply
    never comes: the compute stream parked on the done counter is released by the stall watch
    (a host store of the awaited count into the pinned page) after timeout_s, the channel is
    poisoned, and after reconnect() messages flow again. The stream is polled, never
    synchronized, until released."""
    import time

    from sgl_asap_amd.transport.layout import ChannelPoisoned

    say("loop: dropped message -> stall watch releases the wait, channel poisoned, reconnect")
    experts = make_experts(64)
    with OneGpuAfd(experts, n_max=64, slots=1, timeout_s=0.3, _epoch_override=7) as afd:
        ch, main = afd.channel, torch.cuda.current_stream()
        send = torch.cuda.Stream()
        x, topk = job(12, 950)
        t, held = _send(afd, 0, 0, x, topk, send)
        assert afd.scheduler.serve_pending() == 0 and afd.server.stats["stale_epoch"] == 1
        ch.wait(t, main)
        done = torch.cuda.Event()
        done.record(main)
        deadline = time.monotonic() + 10.0
        while not done.query() and time.monotonic() < deadline:
            time.sleep(0.01)
        if not done.query():  # keep the process able to exit, then fail
            ch.flags.store(ch.g.done_off(0, 0), t.seq)
            pytest.fail("the stall watch did not release the parked wait")
        with pytest.raises(ChannelPoisoned):
            ch.check()
        with pytest.raises(ChannelPoisoned):
            AsapMoE(E, H, I, 0, top_k=K)(x, topk)
        ch._epoch_override = None
        ch.reconnect()
        layer = AsapMoE(E, H, I, 0, top_k=K)
        out = layer(x, topk)
        torch.cuda.synchronize()
        assert np.array_equal(bits16(out), direct(experts, 0, x, topk))


@pytest.mark.parametrize("batch_tokens", [0, 128])
def test_warmup_then_serve(batch_tokens):
    """The F scheduler's warm-up runs every bucket size on two layers (and, with batching, a
    batched call on every F stream), then jobs are served as before."""
    say(f"loop: scheduler warm-up up to 64 tokens, two layers, batch_tokens={batch_tokens}")
    experts = make_experts(64, layers=(0, 1))
    with OneGpuAfd(experts, n_max=64, graph_max_tokens=64, batch_tokens=batch_tokens) as afd:
        assert afd.scheduler.warmup(64) == [1, 2, 4, 8, 16, 32, 64]
        for lid in (0, 1):
            x, topk = job(40, 990 + lid)
            out = AsapMoE(E, H, I, lid, top_k=K)(x, topk)
            torch.cuda.synchronize()
            assert np.array_equal(bits16(out), direct(experts, lid, x, topk))
