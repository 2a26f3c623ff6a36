"""The decode path behind the reference scheduler's call, on the GPU: a model
created like nxt_model_create does (the plugin's nxt_model_init builds the
instance: K/V caches in HBM and the KV-cache index), requests bound by id
and executed like nxt_scheduler_poll executes them
(src/core/scheduler.c:482-486: instance_exec(model->instances, &request, 1)),
and also as whole batches.  Each output is checked against the oracle's
attention (examples/text_gen.c:1284-1310 restated) over the request's
logical K/V history, at the task's tolerance."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import assert_close
from tests.test_gpu_kv_index_decode import Driver
from xllms_amd import backend as B
from xllms_amd import workloads as W

pytestmark = pytest.mark.gpu


def as_model(bits, dtype):
    """fp16 element bits -> a device tensor of the model's element type (fp32:
    the same values, exactly)."""
    if dtype == W.FP32:
        return W.to_torch(np.ascontiguousarray(bits).view(np.float16).astype(np.float32), W.FP32)
    return W.to_torch(bits, dtype)


class Client:
    """Holds each request's token history; K/V and queries come from the
    same prefix-keyed rows as tests/test_gpu_kv_index_decode.py."""

    def __init__(self, model: B.DecodeModel, ref: Driver, dtype):
        self.m, self.ref, self.dtype = model, ref, dtype
        self.hist: dict[str, list] = {}

    def bind(self, rid, new_tokens, rng, release=False, attend=True):
        import torch
        toks = self.hist.setdefault(rid, [])
        start = len(toks)
        toks += [int(t) for t in new_tokens]
        kv = np.stack([self.ref.rows(toks, t) for t in range(start, len(toks))]) \
            if len(new_tokens) else None
        keep = {}
        if kv is not None:
            keep["k"] = as_model(np.ascontiguousarray(kv[:, 0]), self.dtype)
            keep["v"] = as_model(np.ascontiguousarray(kv[:, 1]), self.dtype)
        if attend:
            keep["q_bits"] = rng.standard_normal((self.ref.H, self.ref.D)).astype(np.float16) \
                .view(np.uint16)
            keep["q"] = as_model(keep["q_bits"], self.dtype)
            keep["o"] = torch.empty((self.ref.H, self.ref.D), dtype=W.torch_dtype(self.dtype),
                                    device="cuda")
        rc = self.m.bind(rid, tokens=new_tokens if len(new_tokens) else None,
                         key=keep.get("k"), value=keep.get("v"), query=keep.get("q"),
                         output=keep.get("o"), release=release)
        assert rc == 0
        return keep

    def check(self, rids, binds, what, hist=None):
        """hist: the histories the outputs were computed over (default: now)."""
        import torch
        torch.cuda.synchronize()
        for rid in rids:
            self.ref.live[rid] = (hist or self.hist)[rid]
        q = np.stack([binds[r]["q_bits"] for r in rids])
        want = self.ref.logical_oracle(rids, q)
        got = np.stack([binds[r]["o"].float().cpu().numpy() for r in rids])
        assert_close(got, want, W.FP16, what)
        self.ref.live.clear()


@pytest.mark.parametrize("dtype", [W.FP16, W.FP32], ids=["fp16", "fp32"])
def test_scheduler_style_and_batched_exec(cuda, dtype):
    """fp16 runs the MFMA tile path and the one-launch cascade; fp32 the VALU
    tile path and the two-pass cascade.  Both read each request's query and
    write its output through the exec's row pointers."""
    import torch
    rng = np.random.default_rng(99)
    H, KVH, D, bs = 32, 8, 128, 16
    ref = Driver.__new__(Driver)
    ref.KVH, ref.H, ref.D, ref.bs = KVH, H, D, bs
    ref.scale = 1.0 / np.sqrt(D)
    ref.live, ref._rows = {}, {}
    code = B.NXT_TYPE_FP32 if dtype == W.FP32 else B.NXT_TYPE_FP16
    m = B.DecodeModel(num_blocks=512, num_kv_heads=KVH, block_size=bs, head_size=D,
                      num_heads=H, dtype=code, max_batch_size=16, max_blocks_per_seq=64)
    assert m.status == 0 and m.model.instance_count == 1 and m.model.instances
    c = Client(m, ref, dtype)
    system = list(rng.integers(0, 60, 45))
    rids = [f"req{i}" for i in range(6)]
    # prompts one request per exec, as the scheduler's poll issues them
    for i, rid in enumerate(rids):
        prompt = system + list(rng.integers(0, 60, 20 + 7 * i)) if i < 4 else \
            list(rng.integers(60, 99, 30 + i))
        b = c.bind(rid, prompt, rng)
        assert m.exec([rid]) == 0
        c.check([rid], {rid: b}, f"prefill {rid}")
        if i == 0:
            # make req0's prompt shareable: end it and start it again under a new id
            b = c.bind(rid, [], rng, release=True, attend=False)
            assert m.exec([rid]) == 0
            del c.hist[rid]
            b = c.bind(rid, prompt, rng)
            assert m.exec([rid]) == 0
            c.check([rid], {rid: b}, "re-admitted req0")
    # decode steps: whole batches, then one request per exec
    for step in range(8):
        binds = {rid: c.bind(rid, [int(rng.integers(0, 60))], rng) for rid in rids}
        if step % 2 == 0:
            assert m.exec(rids) == 0
        else:
            for rid in rids:
                assert m.exec([rid]) == 0
        c.check(rids, binds, f"decode step {step}")
    # release half, admit a request that extends a released one's history
    for rid in rids[:3]:
        c.bind(rid, [], rng, release=True, attend=False)
    assert m.exec(rids[:3]) == 0
    ext = c.hist["req1"][:70] + list(rng.integers(0, 60, 9))
    b = c.bind("late", ext, rng)
    assert m.exec(["late"]) == 0
    c.check(["late"], {"late": b}, "late admission")
    # two new requests with a common new prefix in one exec: the second's copy
    # of the partly shared page reads rows the same exec writes
    twin = list(rng.integers(0, 60, 50))
    binds = {"twinA": c.bind("twinA", twin + [1, 2, 3], rng),
             "twinB": c.bind("twinB", twin + [4, 5], rng)}
    assert m.exec(["twinA", "twinB"]) == 0
    c.check(["twinA", "twinB"], binds, "twins admitted together")
    inst = m.model.instances[0]
    assert inst.exec_count > 0 and inst.total_exec_ms > 0
    # errors: unbound request, duplicate id in one batch
    assert m.exec(["nobody"]) == -1
    c.bind("late", [3], rng)
    assert m.exec(["late", "late"]) == -1
    assert m.close() == 0
    torch.cuda.synchronize()


def test_deferred_scheduler_pattern(cuda):
    """Deferred mode (nxt_model_instance_set_deferred): the scheduler's
    one-request execs are queued and run as one batch when flushed -- by
    nxt_model_instance_flush, by binding or executing a queued request again
    (its next step), by a full queue, by switching the mode off and by fini.
    Every flushed output matches the oracle."""
    import torch
    rng = np.random.default_rng(7)
    H, KVH, D, bs = 32, 8, 128, 16
    ref = Driver.__new__(Driver)
    ref.KVH, ref.H, ref.D, ref.bs = KVH, H, D, bs
    ref.scale = 1.0 / np.sqrt(D)
    ref.live, ref._rows = {}, {}
    m = B.DecodeModel(num_blocks=512, num_kv_heads=KVH, block_size=bs, head_size=D,
                      num_heads=H, max_batch_size=4, max_blocks_per_seq=64)
    assert m.status == 0
    c = Client(m, ref, W.FP16)
    rids = [f"d{i}" for i in range(3)]
    shared = list(rng.integers(0, 60, 40))
    assert m.set_deferred(True) == 0
    # prompts: queued, then an explicit flush runs them as one batch
    binds = {rid: c.bind(rid, shared + list(rng.integers(0, 60, 10 + 5 * i)), rng)
             for i, rid in enumerate(rids)}
    for rid in rids:
        assert m.exec([rid]) == 0
    inst = m.model.instances[0]
    assert inst.exec_count == 0  # nothing ran yet
    assert m.flush() == 0
    assert inst.exec_count == 1
    c.check(rids, binds, "deferred prefill")
    # a decode step queued request by request; the next step's first bind
    # flushes it
    binds = {rid: c.bind(rid, [int(rng.integers(0, 60))], rng) for rid in rids}
    for rid in rids:
        assert m.exec([rid]) == 0
    step_hist = {rid: list(c.hist[rid]) for rid in rids}
    nxt = c.bind(rids[0], [int(rng.integers(0, 60))], rng)
    assert inst.exec_count == 2
    c.check(rids, binds, "flushed by the next bind", hist=step_hist)
    # executing a queued request again runs the queue first; the second exec
    # then finds no binding and is refused
    assert m.exec([rids[0]]) == 0
    before = inst.exec_count
    assert m.exec([rids[0]]) == -1
    assert inst.exec_count == before + 1
    c.check([rids[0]], {rids[0]: nxt}, "flushed by a second exec")
    # an unbound request is refused when queued, and nothing runs
    assert m.exec(["nobody"]) == -1
    assert m.flush() == 0 and inst.exec_count == before + 1
    # a full queue (max_batch_size 4) runs at once
    extra = "d3"
    binds = {rid: c.bind(rid, [int(rng.integers(0, 60))], rng) for rid in rids}
    binds[extra] = c.bind(extra, list(rng.integers(60, 99, 33)), rng)
    before = inst.exec_count
    for rid in rids + [extra]:
        assert m.exec([rid]) == 0
    assert inst.exec_count == before + 1
    c.check(rids + [extra], binds, "full queue")
    # switching deferred mode off flushes; fini flushes too
    binds = {rid: c.bind(rid, [int(rng.integers(0, 60))], rng) for rid in rids}
    for rid in rids:
        assert m.exec([rid]) == 0
    assert m.set_deferred(False) == 0
    c.check(rids, binds, "flushed by switching off")
    assert m.set_deferred(True) == 0
    binds = {rid: c.bind(rid, [int(rng.integers(0, 60))], rng) for rid in rids}
    for rid in rids:
        assert m.exec([rid]) == 0
    assert m.close() == 0
    c.check(rids, binds, "flushed by fini")
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype,D", [(W.FP16, 128), (W.FP16, 64), (W.FP32, 128), (W.FP16, 96)],
                         ids=["fp16-d128", "fp16-d64", "fp32-d128", "fp16-d96"])
def test_one_request_decode_steps(cuda, dtype, D):
    """The scheduler's steady state: one instance_exec(.., 1) per running
    request, step after step.  Head sizes 32, 64 and 128 take the one-request
    path that keeps each sequence's length and block table on the device and
    folds the new token in at the merge (96: the general exec).  Prompts of
    15, 16, 17, 31 and 33 tokens put the new tokens on both sides of page
    boundaries; a whole-batch exec in between leaves the device copies stale
    (the next one-request exec uploads them again); a released request's
    handle goes to a new one.  Every output against the oracle."""
    import torch
    rng = np.random.default_rng(5)
    H, KVH, bs = 16, 4, 16
    ref = Driver.__new__(Driver)
    ref.KVH, ref.H, ref.D, ref.bs = KVH, H, D, bs
    ref.scale = 1.0 / np.sqrt(D)
    ref.live, ref._rows = {}, {}
    code = B.NXT_TYPE_FP32 if dtype == W.FP32 else B.NXT_TYPE_FP16
    m = B.DecodeModel(num_blocks=256, num_kv_heads=KVH, block_size=bs, head_size=D,
                      num_heads=H, dtype=code, max_batch_size=8, max_blocks_per_seq=16)
    assert m.status == 0
    c = Client(m, ref, dtype)
    rids = [f"s{i}" for i in range(5)]
    for n, rid in zip([15, 16, 17, 31, 33], rids):
        b = c.bind(rid, list(rng.integers(0, 60, n)), rng)
        assert m.exec([rid]) == 0
        c.check([rid], {rid: b}, f"prefill {rid}")
    for step in range(40):
        binds = {rid: c.bind(rid, [int(rng.integers(0, 60))], rng) for rid in rids}
        if step == 17:
            assert m.exec(rids) == 0
        else:
            for rid in rids:
                assert m.exec([rid]) == 0
        c.check(rids, binds, f"step {step}")
        if step == 25:
            gone = rids.pop(1)
            c.bind(gone, [], rng, release=True, attend=False)
            assert m.exec([gone]) == 0
            del c.hist[gone]
            b = c.bind("new", list(rng.integers(0, 60, 20)), rng)
            assert m.exec(["new"]) == 0
            c.check(["new"], {"new": b}, "admitted after a release")
            rids.append("new")
    assert m.close() == 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("seed", range(12))
def test_random_exec_patterns(cuda, seed):
    """Seeded random serving sessions: head size (32, 64, 96, 128), element
    type (fp16, fp32), block size (16, 32) and GQA shape drawn; prompts that
    share a system prefix or not; every step one new token per live request,
    run as one whole-batch exec, as one exec per request, or as a random
    split into smaller batches; now and then a request ends and a new one is
    admitted (its handle reused).  One-request execs take the path that keeps
    each sequence's table and length on the device where the head size
    allows, and every mix of the patterns must leave those copies right.
    Every output against the oracle."""
    import torch
    rng = np.random.default_rng(7000 + seed)
    D = int(rng.choice([32, 64, 96, 128]))
    dtype = W.FP32 if rng.random() < 0.3 else W.FP16
    bs = int(rng.choice([16, 32]))
    H, KVH = [(8, 2), (16, 4), (8, 8)][int(rng.integers(0, 3))]
    ref = Driver.__new__(Driver)
    ref.KVH, ref.H, ref.D, ref.bs = KVH, H, D, bs
    ref.scale = 1.0 / np.sqrt(D)
    ref.live, ref._rows = {}, {}
    code = B.NXT_TYPE_FP32 if dtype == W.FP32 else B.NXT_TYPE_FP16
    m = B.DecodeModel(num_blocks=512, num_kv_heads=KVH, block_size=bs, head_size=D,
                      num_heads=H, dtype=code, max_batch_size=8, max_blocks_per_seq=160 // bs)
    assert m.status == 0
    c = Client(m, ref, dtype)
    system = list(rng.integers(0, 50, int(rng.integers(1, 40))))
    count = [0]

    def admit():
        rid = f"q{count[0]}"
        count[0] += 1
        tail = list(rng.integers(0, 50, int(rng.integers(1, 30))))
        prompt = system + tail if rng.random() < 0.5 else tail
        b = c.bind(rid, prompt, rng)
        assert m.exec([rid]) == 0
        c.check([rid], {rid: b}, f"seed {seed}: admit {rid}")
        return rid

    live = [admit() for _ in range(int(rng.integers(2, 6)))]
    print(f"case seed={seed} d={D} {'fp32' if dtype == W.FP32 else 'fp16'} bs={bs} H={H} "
          f"KVH={KVH} requests={len(live)}", flush=True)
    for step in range(30):
        binds = {rid: c.bind(rid, [int(rng.integers(0, 50))], rng) for rid in live}
        pattern = int(rng.integers(0, 3))
        if pattern == 0:
            assert m.exec(live) == 0
        elif pattern == 1:
            for rid in live:
                assert m.exec([rid]) == 0
        else:
            order = list(rng.permutation(live))
            while order:
                k = int(rng.integers(1, len(order) + 1))
                assert m.exec(order[:k]) == 0
                order = order[k:]
        c.check(live, binds, f"seed {seed}: step {step} pattern {pattern}")
        if rng.random() < 0.15 and len(live) > 1:
            gone = live.pop(int(rng.integers(0, len(live))))
            c.bind(gone, [], rng, release=True, attend=False)
            assert m.exec([gone]) == 0
            del c.hist[gone]
            live.append(admit())
    assert m.close() == 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype,D,bs", [(W.FP16, 128, 16), (W.FP32, 64, 32), (W.FP16, 96, 16)],
                         ids=["fp16-d128-bs16", "fp32-d64-bs32", "fp16-d96-bs16"])
def test_batch_tables_kept_on_device(cuda, dtype, D, bs):
    """Whole-batch execs keep the batch's block tables on the device: an exec
    over the same requests in the same order, whose sequences grew only by
    its own appends, stores just the entries of the pages those appends
    opened.  Steps append 1 to 40 tokens per request (pages opened on every
    kind of boundary, and rows outgrowing their spare entries, which uploads
    the tables again); between them, requests grow outside the batch (a
    K/V-only exec, a one-request exec), the order changes and changes back,
    a deferred-mode flush runs the same batch, and a released request's
    handle goes to a new one.  Every output against the oracle."""
    import torch
    rng = np.random.default_rng(17)
    H, KVH = 16, 4
    ref = Driver.__new__(Driver)
    ref.KVH, ref.H, ref.D, ref.bs = KVH, H, D, bs
    ref.scale = 1.0 / np.sqrt(D)
    ref.live, ref._rows = {}, {}
    code = B.NXT_TYPE_FP32 if dtype == W.FP32 else B.NXT_TYPE_FP16
    m = B.DecodeModel(num_blocks=1024, num_kv_heads=KVH, block_size=bs, head_size=D,
                      num_heads=H, dtype=code, max_batch_size=8,
                      max_blocks_per_seq=2048 // bs)
    assert m.status == 0
    c = Client(m, ref, dtype)
    rids = [f"t{i}" for i in range(5)]
    for n, rid in zip([1, bs - 1, bs, bs + 1, 3 * bs + 7], rids):
        b = c.bind(rid, list(rng.integers(0, 60, n)), rng)
        assert m.exec([rid]) == 0
        c.check([rid], {rid: b}, f"prefill {rid}")
    order = list(rids)
    for step in range(48):
        # (the first 20 steps grow fast, so rows outgrow their spare entries)
        grow = [int(rng.choice([20, 40] if step < 20 else [1, 1, 2, 7, 20, 40])) for _ in order]
        binds = {rid: c.bind(rid, list(rng.integers(0, 60, k)), rng)
                 for rid, k in zip(order, grow)}
        if step < 20:
            assert m.exec(order) == 0
        elif step % 12 == 5:  # the same batch through deferred mode's flush
            assert m.set_deferred(True) == 0
            for rid in order:
                assert m.exec([rid]) == 0
            assert m.flush() == 0
            assert m.set_deferred(False) == 0
        else:
            assert m.exec(order) == 0
        c.check(order, binds, f"step {step} grow {grow}")
        if step < 20:
            continue
        if step % 12 == 3:  # one request grows outside the batch: K/V only
            rid = order[int(rng.integers(0, len(order)))]
            c.bind(rid, list(rng.integers(0, 60, 3)), rng, attend=False)
            assert m.exec([rid]) == 0
        elif step % 12 == 7:  # ... or by a one-request decode step
            rid = order[int(rng.integers(0, len(order)))]
            b = c.bind(rid, [int(rng.integers(0, 60))], rng)
            assert m.exec([rid]) == 0
            c.check([rid], {rid: b}, f"step {step}: one-request exec of {rid}")
        elif step % 12 == 9:  # another order, and back two steps later
            order = list(rng.permutation(order))
        elif step % 12 == 11:
            order = sorted(order, key=lambda r: (len(r), r))
        if step == 30:
            gone = order.pop(2)
            c.bind(gone, [], rng, release=True, attend=False)
            assert m.exec([gone]) == 0
            del c.hist[gone]
            b = c.bind("late", list(rng.integers(0, 60, 2 * bs + 3)), rng)
            assert m.exec(["late"]) == 0
            c.check(["late"], {"late": b}, "admitted after a release")
            order.insert(2, "late")
    assert m.close() == 0
    torch.cuda.synchronize()
