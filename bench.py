#!/usr/bin/env python3
"""Benchmark of the MI355X paged-decode attention (one GPU).

Default workload: BASELINE config 2, the Llama-3-8B GQA ragged decode batch
(32 q / 8 kv heads, d=128, fp16, bs=16, B=64, L ~ U[512, 4096], 2x page pool
with garbage).  A step is one call of the reference entry point
nxt_paged_attention over the whole batch, with every input already resident in
HBM.  Steps rotate over several independent copies of the K/V pool (>= 3 and
>= 768 MB in total) so no step is served from the 256 MB MALL of the previous
one.  The reference bench's shape flags (--batch --ctx --heads --kv-heads
--head-size --dtype, tests/test_attention_bench.c:421-435) select its
workload instead: every sequence at --ctx tokens (defaults B 16, ctx 1024,
32 q / 8 kv heads, d 128, fp16), seeded N(0,1) data and a permuted table.

Prints ONE JSON line:
  value        seqs/s = num_seqs / (GPU time per step), whole job on 1 GPU
  roofline     algorithmic bytes of one launch / average duration of the
               partition kernel (HIP events stamped with each launch's start
               and end on its stream, over K further steps kept apart from the
               K timed steps that give `value`), against 8 TB/s;
               `traffic` = HBM bytes per launch from the committed rocprofv3
               PMC summary for this workload (profiles/), else null
               step_frac: algorithmic bytes / whole step time (partition and merge
               launches, back to back), against 8 TB/s
  measured_peak the ceilings measured in the same run: the batch's own K/V
               tiles streamed with the kernel's loads and no arithmetic
               (xllm_stream_probe), and a plain 1 GiB device copy; the kernel's
               and the step's rate as fractions of the former
  cpu_baseline the oracle (C restatement of the reference CPU attention)
               on the host cores, all threads; single-thread figure alongside
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "paged-decode attn seqs/s + achieved HBM GB/s (% peak), Llama-3-8B GQA shape"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class HipEvents:
    """hipEvent_t handles through the HIP runtime torch already loaded."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
        self.events = []

    def create(self) -> int:
        ev = ctypes.c_void_p()
        rc = self.hip.hipEventCreate(ctypes.byref(ev))
        if rc != 0:
            raise RuntimeError(f"hipEventCreate failed: {rc}")
        self.events.append(ev.value)
        return ev.value

    def record(self, ev: int, stream: int) -> None:
        rc = self.hip.hipEventRecord(ev, stream)
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed: {rc}")

    def elapsed_ms(self, a: int, b: int) -> float:
        ms = ctypes.c_float()
        rc = self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed: {rc}")
        return ms.value

    def sync(self, stream: int) -> None:
        rc = self.hip.hipStreamSynchronize(stream)
        if rc != 0:
            raise RuntimeError(f"hipStreamSynchronize failed: {rc}")

    def destroy_all(self) -> None:
        for ev in self.events:
            self.hip.hipEventDestroy(ev)
        self.events.clear()


def load_traffic(workload_name: str):
    """HBM bytes per launch of the partition kernel from the committed PMC
    summary (profiles/<workload>_pmc.json), or None."""
    path = os.path.join(ROOT, "profiles", f"{workload_name}_pmc.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        d = json.load(f)
    return d.get("hbm_bytes_per_launch")


def tile_descriptors(wl, distinct: bool = False):
    """The batch's 16-token K/V tiles in the decode's order (sequence, kv
    head, tile) as xllm_stream_probe descriptors: byte offset << 5 | valid
    rows.  distinct: each (physical page, kv head) once, with the most valid
    rows any sequence reads from it (the compulsory tiles of a shared-prefix
    batch)."""
    import numpy as np
    bs, eb, D = wl.block_size, wl.elem_bytes, wl.head_size
    if bs != 16:
        return None
    seen = {}
    parts = []
    for s, L in enumerate(wl.seq_lens):
        L = int(L)
        nt = -(-L // 16)
        if nt == 0:
            continue
        blk = wl.block_tables[s, :nt].astype(np.int64)
        rows = np.minimum(16, L - 16 * np.arange(nt)).astype(np.int64)
        keep = blk >= 0
        blk, rows = blk[keep], rows[keep]
        if distinct:
            for b, r in zip(blk.tolist(), rows.tolist()):
                seen[b] = max(seen.get(b, 0), r)
            continue
        for h in range(wl.num_kv_heads):
            off = (blk * wl.kv_block_stride + h * wl.kv_head_stride) * eb
            parts.append((off << 5) | rows)
    if distinct:
        blk = np.array(sorted(seen), dtype=np.int64)
        rows = np.array([seen[b] for b in blk.tolist()], dtype=np.int64)
        for h in range(wl.num_kv_heads):
            off = (blk * wl.kv_block_stride + h * wl.kv_head_stride) * eb
            parts.append((off << 5) | rows)
    desc = np.concatenate(parts) if parts else np.zeros(0, dtype=np.int64)
    kv_bytes = int((desc & 31).sum()) * D * eb * 2
    return desc, kv_bytes


def pattern_peak(wl, kpools, vpools, waves: int, steps: int, distinct: bool = False):
    """Rate at which this batch's K/V tiles stream with the decode kernel's
    access pattern and no arithmetic (xllm_stream_probe over the same pools,
    rotated like the timed steps): GB/s of K/V bytes, or None."""
    import torch
    from xllms_amd import _lib
    tb = 16 * wl.head_size * wl.elem_bytes
    got = tile_descriptors(wl, distinct)
    if got is None or tb not in (1024, 2048, 4096):
        return None
    desc, kv_bytes = got
    lib = _lib.stream_probe()
    d_desc = torch.from_numpy(desc).to("cuda")
    sink = torch.empty(waves * 64, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def launch(i):
        rc = lib.xllm_stream_probe(kpools[i % len(kpools)].data_ptr(),
                                   vpools[i % len(vpools)].data_ptr(), d_desc.data_ptr(),
                                   int(desc.size), tb, waves, sink.data_ptr(), stream)
        if rc != 0:
            raise RuntimeError("xllm_stream_probe failed")

    for i in range(20):
        launch(i)
    ev = HipEvents()
    a, b = ev.create(), ev.create()
    torch.cuda.synchronize()
    ev.record(a, stream)
    for i in range(steps):
        launch(i)
    ev.record(b, stream)
    torch.cuda.synchronize()
    ms = ev.elapsed_ms(a, b) / steps
    ev.destroy_all()
    return {"gbs": round(kv_bytes / (ms / 1e3) / 1e9, 1), "us": round(ms * 1e3, 2),
            "kv_bytes": kv_bytes, "tiles": int(desc.size), "waves": waves}


def device_copy_peak(mib: int = 1024, steps: int = 10) -> dict:
    """A plain device-to-device copy (torch copy_, the runtime's copy kernel)
    of `mib` MiB: bytes read + written per second."""
    import torch
    n = mib * 2**20 // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    stream = torch.cuda.current_stream().cuda_stream
    ev = HipEvents()
    a, b = ev.create(), ev.create()
    torch.cuda.synchronize()
    ev.record(a, stream)
    for _ in range(steps):
        dst.copy_(src)
    ev.record(b, stream)
    torch.cuda.synchronize()
    ms = ev.elapsed_ms(a, b) / steps
    ev.destroy_all()
    del src, dst
    torch.cuda.empty_cache()
    return {"gbs": round(2 * n * 4 / (ms / 1e3) / 1e9, 1), "bytes_moved": 2 * n * 4,
            "us": round(ms * 1e3, 2)}


def partition_kernel_name(wl) -> str:
    """Kernel that streams K/V for this workload: the MFMA tile kernel serves
    fp16/bf16 pages with head_size % 32 == 0 and block_size >= 16, the VALU
    tile kernel everything else (same rule as use_mfma in paged_decode_api.cpp);
    on the VALU path, batches of at most one segment per CU with groups of
    at most 2 heads run one round of workgroups over the segments, 1, 2 or 4
    per segment of at most 128 tiles each (the seg_split rule in
    paged_decode_api.cpp)."""
    import torch
    from xllms_amd import workloads as W
    mfma = wl.kv_dtype != W.FP32 and wl.head_size % 32 == 0 and wl.block_size >= 16
    if mfma:
        return "paged_decode_partition_mfma_kernel"
    group = wl.num_heads // wl.num_kv_heads
    lanes = 1
    while lanes < wl.head_size * wl.elem_bytes // 16:
        lanes *= 2
    rows = 64 // lanes  # tile rows per 16-byte load
    tile = 4 * rows
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    max_ctx = wl.max_num_blocks_per_seq * wl.block_size
    segs = wl.num_seqs * wl.num_kv_heads
    if group <= 2 and wl.block_size >= rows and segs <= cus:
        tiles, seg_bytes, split = -(-max_ctx // tile), max_ctx * wl.head_size * wl.elem_bytes * 2, 1
        while split < 4 and segs * split * 2 <= cus and (seg_bytes // (split * 2) >= 160 << 10 or
                                                         tiles > split * 128):
            split *= 2
        if tiles <= split * 128:
            return "paged_decode_segment_kernel"
    return "paged_decode_partition_kernel"


def cpu_baseline(wl, budget_s: float) -> dict:
    """Time the oracle on the host: all threads, then one thread, each on a
    sample of about budget_s / 2 seconds, as many whole copies of the batch
    as fit, or else its leading sequences.  The sample is sized from a probe
    on leading sequences that grows until it takes >= 50 ms, by tokens (a
    batch whose first sequences are short, like config 5's, would otherwise
    be sampled far past the budget).  The rate is in this batch's sequences
    per second: the sample's tokens per second over the batch's tokens per
    sequence (for whole copies, exactly sequences per second)."""
    import numpy as np
    from oracle import oracle as O
    threads = O.lib().oracle_num_threads()
    cum = np.cumsum(np.maximum(np.asarray(wl.seq_lens, dtype=np.int64), 0))
    total = max(1, int(cum[-1]))
    tok_per_seq = total / wl.num_seqs
    res = {}
    for name, prec, nthr in (("all", "mt", threads), ("single", "f32", 1)):
        k = 1
        while True:
            t0 = time.perf_counter()
            O.run_workload(wl, precision=prec, threads=nthr, seqs=slice(0, k))
            dt = max(time.perf_counter() - t0, 1e-6)
            if dt >= 0.05 or k >= wl.num_seqs:
                break
            k = min(wl.num_seqs, 4 * k)
        per_tok = dt / max(1, int(cum[k - 1]))
        budget_tok = budget_s / 2 / per_tok
        if budget_tok >= total:
            nseq, reps = wl.num_seqs, int(max(1, budget_tok // total))
        else:
            nseq, reps = int(max(1, np.searchsorted(cum, budget_tok, side="right"))), 1
        t0 = time.perf_counter()
        for _ in range(reps):
            O.run_workload(wl, precision=prec, threads=nthr, seqs=slice(0, nseq))
        dt = time.perf_counter() - t0
        toks = int(cum[nseq - 1]) * reps
        res[name] = {"seqs": nseq * reps, "tokens": toks, "seconds": dt, "threads": nthr,
                     "seqs_per_s": toks / dt / tok_per_seq}
    return res


def bench_kv_append(args) -> int:
    """KV append on the workload's shape.  Prefill form: all tokens of the
    batch (their K/V rows gathered from the pool, so writing them back must
    leave the pool unchanged: the check) written to their slots; decode form:
    one new token per sequence.  Algorithmic bytes = rows read + rows written
    + 4 B per slot."""
    import numpy as np
    import torch
    from xllms_amd import paged_attention as PA
    from xllms_amd import workloads as W

    wl = workload_from_args(args)
    dw = W.upload(wl)
    bs, kvh, d = wl.block_size, wl.num_kv_heads, wl.head_size
    slots = []
    for s_, L in enumerate(wl.seq_lens):
        for t in range(int(L)):
            slots.append(int(wl.block_tables[s_, t // bs]) * bs + t % bs)
    slots = np.asarray(slots, dtype=np.int32)
    n = len(slots)
    sl = torch.from_numpy(slots).cuda()
    blk = sl.long() // bs
    off = sl.long() % bs
    key = dw.key_cache[blk, :, off, :].contiguous()        # [n, kvh, d]
    value = dw.value_cache[blk, :, off, :].contiguous()
    k_before = dw.key_cache.clone()
    v_before = dw.value_cache.clone()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream().cuda_stream
    lib = PA._lib.backend()
    a = (dw.key_cache.data_ptr(), dw.value_cache.data_ptr(), key.data_ptr(), value.data_ptr(),
         sl.data_ptr(), n, kvh, d, bs, wl.kv_block_stride, wl.kv_head_stride, wl.kv_dtype, stream)
    for _ in range(args.warmup):
        lib.nxt_paged_kv_write_slots(*a)
    ev = HipEvents()
    e0, e1 = ev.create(), ev.create()
    torch.cuda.synchronize()
    ev.record(e0, stream)
    for _ in range(args.steps):
        lib.nxt_paged_kv_write_slots(*a)
    ev.record(e1, stream)
    torch.cuda.synchronize()
    st, msg = PA.last_status()
    if st != 0:
        raise RuntimeError(f"kv append failed: {msg}")
    ms = ev.elapsed_ms(e0, e1) / args.steps
    ibits = torch.int32 if wl.kv_dtype == W.FP32 else torch.int16   # the pool holds NaN sentinels
    unchanged = bool(torch.equal(dw.key_cache.view(ibits), k_before.view(ibits)) and
                     torch.equal(dw.value_cache.view(ibits), v_before.view(ibits)))
    row_bytes = kvh * d * wl.elem_bytes
    alg = 2 * n * row_bytes * 2 + 4 * n
    gbs = alg / (ms / 1e3) / 1e9
    # decode step: one token per sequence, at its last position
    pos = torch.from_numpy((wl.seq_lens - 1).astype(np.int32)).cuda()
    kd = key[:wl.num_seqs].contiguous()
    vd = value[:wl.num_seqs].contiguous()
    ad = (dw.key_cache.data_ptr(), dw.value_cache.data_ptr(), kd.data_ptr(), vd.data_ptr(),
          dw.block_tables.data_ptr(), pos.data_ptr(), wl.num_seqs, kvh, d,
          wl.max_num_blocks_per_seq, bs, wl.kv_block_stride, wl.kv_head_stride, wl.kv_dtype, stream)
    for _ in range(args.warmup):
        lib.nxt_paged_kv_append(*ad)
    torch.cuda.synchronize()
    ev.record(e0, stream)
    for _ in range(args.steps):
        lib.nxt_paged_kv_append(*ad)
    ev.record(e1, stream)
    torch.cuda.synchronize()
    dms = ev.elapsed_ms(e0, e1) / args.steps
    ev.destroy_all()
    log(f"[bench] kv append: {n} tokens in {ms * 1e3:.1f} us = {gbs:.0f} GB/s "
        f"({gbs / HBM_PEAK_GBS:.1%} of 8 TB/s); decode step ({wl.num_seqs} tokens) "
        f"{dms * 1e3:.2f} us; pool unchanged after write-back: {unchanged}")
    print(json.dumps({
        "metric": "paged KV append GB/s (prefill form) + decode-step latency",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "higher_is_better": True,
        "dtype": {W.FP16: "fp16", W.BF16: "bf16", W.FP32: "fp32"}[wl.kv_dtype],
        "data": "synthetic (rows gathered from the seeded pool)",
        "config": {"workload": wl.name, "tokens": n, "num_kv_heads": kvh, "head_size": d,
                   "block_size": bs},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "paged_kv_append_kernel", "kernel_avg_us": round(ms * 1e3, 2)},
        "decode_step_us": round(dms * 1e3, 2), "decode_tokens": wl.num_seqs,
        "check": {"pool_unchanged_after_write_back": unchanged}}), flush=True)
    return 0 if unchanged else 1


ACT_OPS = {"silu_and_mul": 1, "mul_and_silu": 2, "gelu_and_mul": 3, "gelu_tanh_and_mul": 4,
           "gelu": 5, "silu": 6}


def bench_activation(args) -> int:
    """The MLP activation of the Llama-3-8B shape (intermediate size 14336,
    fp16) over a prefill chunk of --act-tokens tokens, through the
    reference-named entry point (nxt_silu_and_mul etc.).  Algorithmic bytes
    per launch = input (2d or d elements per token) + output (d per token).
    Steps alternate between two input/output pairs (each > the 256 MB MALL at
    the default size).  Also times the decode-sized call (64 tokens)."""
    import numpy as np
    import torch
    from oracle import oracle as O
    from xllms_amd import activation as A
    from xllms_amd import paged_attention as PA

    op = ACT_OPS[args.activation]
    entry = {v: k for k, v in A.ENTRY_POINTS.items()}[op]
    gated = A.is_gated(op)
    n, d = args.act_tokens, 14336
    cols = 2 * d if gated else d
    gen = torch.Generator(device="cuda").manual_seed(20260100 + op)
    ins = [(torch.randn((n, cols), generator=gen, device="cuda") * 3).half() for _ in range(2)]
    outs = [torch.empty((n, d), dtype=torch.float16, device="cuda") for _ in range(2)]
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream().cuda_stream
    lib = PA._lib.backend()
    fn = getattr(lib, entry)
    call = [(outs[i].data_ptr(), ins[i].data_ptr(), n, d, 2, stream) for i in range(2)]
    for i in range(args.warmup):
        fn(*call[i % 2])
    # one kernel per call: the launches run back to back between two events,
    # so the average is the kernel's duration plus the short dispatch gap
    ev = HipEvents()
    e0, e1 = ev.create(), ev.create()
    torch.cuda.synchronize()
    ev.record(e0, stream)
    for i in range(args.steps):
        fn(*call[i % 2])
    ev.record(e1, stream)
    torch.cuda.synchronize()
    st, msg = PA.last_status()
    if st != 0:
        raise RuntimeError(f"activation failed: {msg}")
    avg_ms = ev.elapsed_ms(e0, e1) / args.steps
    alg = n * (cols + d) * 2
    gbs = alg / (avg_ms / 1e3) / 1e9
    # decode-sized call: 64 tokens
    dn = 64
    for _ in range(args.warmup):
        fn(outs[0].data_ptr(), ins[0].data_ptr(), dn, d, 2, stream)
    torch.cuda.synchronize()
    ev.record(e0, stream)
    for _ in range(args.steps):
        fn(outs[0].data_ptr(), ins[0].data_ptr(), dn, d, 2, stream)
    ev.record(e1, stream)
    torch.cuda.synchronize()
    dec_us = ev.elapsed_ms(e0, e1) / args.steps * 1e3
    ev.destroy_all()
    # check 16 rows against the oracle: within 2 ulps, >= 99% bit-identical
    fn(outs[0].data_ptr(), ins[0].data_ptr(), n, d, 2, stream)
    torch.cuda.synchronize()
    rows = np.linspace(0, n - 1, 16).astype(int)
    xb = ins[0][rows].view(torch.int16).cpu().numpy().view(np.uint16)
    got = outs[0][rows].view(torch.int16).cpu().numpy().astype(np.int64)
    ref = O.activation(op, xb, O.FP16).view(np.int16).astype(np.int64)
    mono = lambda b: np.where(b < 0, -(b & 0x7FFF), b)  # noqa: E731
    dist = np.abs(mono(got) - mono(ref))
    check = {"rows_checked": int(rows.size), "max_ulp": int(dist.max()),
             "identical": round(float((dist == 0).mean()), 5)}
    ok = check["max_ulp"] <= 2 and check["identical"] >= 0.99
    cpu = None
    if not args.no_cpu_baseline:
        threads = O.lib().oracle_num_threads()
        res = {}
        for name, nthr in (("all", threads), ("single", 1)):
            probe = xb[:2]
            t0 = time.perf_counter()
            O.activation(op, probe, O.FP16, threads=nthr)
            per_tok = max(time.perf_counter() - t0, 1e-6) / 2
            ntok = int(max(2, min(n, args.cpu_budget / 2 / per_tok)))
            sample = ins[0][:ntok].view(torch.int16).cpu().numpy().view(np.uint16)
            t0 = time.perf_counter()
            O.activation(op, sample, O.FP16, threads=nthr)
            dt = time.perf_counter() - t0
            res[name] = {"tokens": ntok, "seconds": dt, "threads": nthr}
        a = res["all"]
        cpu = {"value": round(a["tokens"] / a["seconds"], 1), "unit": "tokens/s",
               "cores": a["threads"], "kind": "port",
               "sample": f"oracle/activation_oracle.c (C restatement of activation_kernels.cu:"
                         f"24-134, gcc -O2, OpenMP over tokens) on {a['tokens']} tokens of this "
                         f"batch in {a['seconds']:.1f}s",
               "gbs_all_threads": round(a["tokens"] * (cols + d) * 2 / a["seconds"] / 1e9, 2),
               "single_thread": {"value": round(res["single"]["tokens"] /
                                                res["single"]["seconds"], 1),
                                 "cores": 1, "sample": f"{res['single']['tokens']} tokens in "
                                                       f"{res['single']['seconds']:.1f}s"}}
    log(f"[bench] {entry} {n}x{d} fp16: {avg_ms * 1e3:.1f} us = "
        f"{gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of 8 TB/s); decode call ({dn} tokens) "
        f"{dec_us:.2f} us; check {check}")
    print(json.dumps({
        "metric": f"{args.activation} tokens/s + achieved HBM GB/s (% peak), Llama-3-8B MLP shape",
        "value": round(n / (avg_ms / 1e3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(avg_ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded N(0,1)*3 activations)",
        "config": {"workload": f"llama3-8b-mlp-{args.activation}-fp16", "tokens": n,
                   "intermediate_size": d, "entry_point": entry},
        "algorithmic_bytes": alg,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic(f"llama3-8b-mlp-{args.activation}-fp16"),
                     "kernel": "activation_vec_kernel", "kernel_avg_us": round(avg_ms * 1e3, 2)},
        "decode_call_us": round(dec_us, 2), "decode_tokens": dn,
        "cpu_baseline": cpu, "check": check}), flush=True)
    return 0 if ok else 1


def bare_decode_step_us(wl, steps: int, warmup: int) -> float:
    """Step time of one nxt_paged_attention call over the workload, with its
    inputs resident in HBM (>= 3 rotated K/V pools, HIP events around `steps`
    back-to-back calls): the bare attention of a batch the serving path also
    runs."""
    import torch
    from xllms_amd import paged_attention as PA
    from xllms_amd import workloads as W
    dw = W.upload(wl, "cuda")
    pool_bytes = 2 * dw.key_cache.numel() * dw.key_cache.element_size()
    pools = max(3, -(-768 * 2**20 // pool_bytes))
    kp, vp = [dw.key_cache], [dw.value_cache]
    for _ in range(pools - 1):
        kp.append(dw.key_cache.clone())
        vp.append(dw.value_cache.clone())
    stream = torch.cuda.current_stream().cuda_stream
    lib = PA._lib.backend()
    fn = lib.nxt_paged_attention_ex
    calls = [(dw.out.data_ptr(), dw.query.data_ptr(), k.data_ptr(), v.data_ptr(),
              dw.block_tables.data_ptr(), dw.seq_lens.data_ptr(), wl.num_seqs, wl.num_heads,
              wl.head_size, wl.num_kv_heads, ctypes.c_float(wl.scale), wl.max_num_blocks_per_seq,
              wl.block_size, wl.elem_bytes, wl.kv_block_stride, wl.kv_head_stride, stream,
              wl.kv_dtype, 0) for k, v in zip(kp, vp)]
    for i in range(warmup):
        fn(*calls[i % pools])
    ev = HipEvents()
    a, b = ev.create(), ev.create()
    torch.cuda.synchronize()
    ev.record(a, stream)
    for i in range(steps):
        fn(*calls[i % pools])
    ev.record(b, stream)
    torch.cuda.synchronize()
    st, msg = PA.last_status()
    if st != 0:
        raise RuntimeError(f"bare decode step failed: {msg}")
    us = ev.elapsed_ms(a, b) / steps * 1e3
    ev.destroy_all()
    del dw, kp, vp, calls
    torch.cuda.empty_cache()
    return us


def launch_floor(wl1, reps: int = 200) -> dict:
    """What a synchronous exec cannot go below on this runtime, timed on the
    host from Python (each figure includes one ctypes call, ~0.5 us): one
    near-empty kernel launch followed by hipStreamSynchronize, and one bare
    nxt_paged_attention call over the one-sequence workload wl1 followed by
    hipStreamSynchronize.  Medians of `reps`."""
    import numpy as np
    import torch
    from xllms_amd import _lib
    from xllms_amd import paged_attention as PA
    from xllms_amd import workloads as W
    stream = torch.cuda.current_stream().cuda_stream
    ev = HipEvents()
    probe = _lib.stream_probe()
    dummy = torch.zeros(64, dtype=torch.int64, device="cuda")
    sink = torch.empty(64 * 64, dtype=torch.int32, device="cuda")
    def empty():
        # no tiles: 16 workgroups that only store their word
        if probe.xllm_stream_probe(dummy.data_ptr(), dummy.data_ptr(), dummy.data_ptr(), 0, 4096,
                                   64, sink.data_ptr(), stream) != 0:
            raise RuntimeError("xllm_stream_probe failed")
    dw = W.upload(wl1, "cuda")
    lib = PA._lib.backend()
    a = (dw.out.data_ptr(), dw.query.data_ptr(), dw.key_cache.data_ptr(),
         dw.value_cache.data_ptr(), dw.block_tables.data_ptr(), dw.seq_lens.data_ptr(),
         wl1.num_seqs, wl1.num_heads, wl1.head_size, wl1.num_kv_heads, ctypes.c_float(wl1.scale),
         wl1.max_num_blocks_per_seq, wl1.block_size, wl1.elem_bytes, wl1.kv_block_stride,
         wl1.kv_head_stride, stream, wl1.kv_dtype, 0)
    def attention():
        lib.nxt_paged_attention_ex(*a)
    out = {}
    for key, fn in (("empty_launch_sync_us", empty), ("one_request_attention_sync_us", attention)):
        for _ in range(20):
            fn()
            ev.sync(stream)
        t = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ev.sync(stream)
            t.append(time.perf_counter() - t0)
        out[key] = round(float(np.median(t)) * 1e6, 1)
    st, msg = PA.last_status()
    if st != 0:
        raise RuntimeError(f"attention call failed: {msg}")
    out["one_request_tokens"] = int(wl1.seq_lens[0])
    ev.destroy_all()
    return out


def bench_serve(args) -> int:
    """Decode steps through the plugin's model instance: the path the
    reference scheduler's poll reaches (src/core/scheduler.c:482-486,
    instance_exec).  The config's prompts are admitted first (their K/V
    written through the KV-cache index; config 5's shared prefixes are
    matched and shared), then each timed step binds one new token, its K/V
    rows and a query for every request and runs one exec over the whole
    batch: index work on the host, staging uploads, the K/V write, the decode
    attention (prefix-aware when the batch shares prefixes) and the output
    scatter, waited for.  The binding calls and the request array (Python)
    are outside the timed region; the native exec call is timed with the host
    clock.  XLLM_HIP_EXEC_TRACE=1 prints each exec's phase times.  With
    --per-request the same steps also run as one instance_exec(.., 1) per
    request in deferred mode with one flush per step (taking turns with the
    whole-batch execs), and then as many steps run as one synchronous
    instance_exec(.., 1) per request (the reference scheduler's pattern)."""
    import numpy as np
    import torch
    from xllms_amd import backend as B
    from xllms_amd import workloads as W

    name, H, KVH, D, kv_dtype, prompts = W.serve_prompts(args.config)
    tdt = W.torch_dtype(kv_dtype)
    nreq, bs = len(prompts), 16
    lens = np.array([len(p) for p in prompts])
    # every timed mode appends one token per request per step
    phases = 3 if args.per_request else 1
    grow = phases * (args.warmup + args.steps) + 1
    pages = int(sum(-(-(int(L) + grow) // bs) for L in lens))
    max_blocks = int(-(-(int(lens.max()) + grow) // bs))
    dtype_code = {W.FP16: B.NXT_TYPE_FP16, W.BF16: B.NXT_TYPE_BF16_HIP,
                  W.FP32: B.NXT_TYPE_FP32}[kv_dtype]
    m = B.DecodeModel(num_blocks=pages + 64, num_kv_heads=KVH, block_size=bs, head_size=D,
                      num_heads=H, dtype=dtype_code, max_batch_size=nreq,
                      max_blocks_per_seq=max_blocks)
    if m.status != 0:
        raise RuntimeError("nxt_model_init failed")
    rids = [f"r{i}" for i in range(nreq)]
    gen = torch.Generator(device="cuda").manual_seed(5)
    t_prefill = time.perf_counter()
    for i, (rid, prompt) in enumerate(zip(rids, prompts)):
        kv = torch.randn((2, len(prompt), KVH, D), generator=gen, device="cuda").to(tdt)
        assert m.bind(rid, tokens=prompt, key=kv[0], value=kv[1]) == 0
        if m.exec([rid]) != 0:
            raise RuntimeError(f"prefill of {rid} failed")
    t_prefill = time.perf_counter() - t_prefill
    kv_new = torch.randn((2, nreq, KVH, D), generator=gen, device="cuda").to(tdt)
    q = torch.randn((nreq, H, D), generator=gen, device="cuda").to(tdt)
    out = torch.empty_like(q)
    rng = np.random.default_rng(11)
    batch = m.requests(rids)
    singles = [m.requests([rid]) for rid in rids]

    # Each step binds every request's new token, its K/V rows and its query
    # and output rows.  The bind calls go to the C entry point with prebuilt
    # arguments (one NxtDecodeIo per request, the buffers fixed, the token
    # written in place; the bind copies it), as the exec calls below do: a
    # scheduler in C binds in a few us per request, and between its steps
    # the device idles for about that long, not for the ~1 ms a Python
    # binding loop takes (after which the next exec runs slower: the GPU's
    # idle power state).
    tok_buf = np.zeros(nreq, dtype=np.int32)
    ios = []
    for i in range(nreq):
        io = B.NxtDecodeIo(struct_size=ctypes.sizeof(B.NxtDecodeIo), num_tokens=1,
                           token_ids=tok_buf.ctypes.data + 4 * i, key=kv_new[0, i].data_ptr(),
                           value=kv_new[1, i].data_ptr(), query=q[i].data_ptr(),
                           output=out[i].data_ptr())
        ios.append(io)
    bind_args = [(rid.encode(), ctypes.byref(io)) for rid, io in zip(rids, ios)]
    bind_fn = m.dl.nxt_model_instance_bind

    def bind_step():
        tok_buf[:] = rng.integers(0, 32000, nreq)
        for rid_b, io_ref in bind_args:
            if bind_fn(m.instance, rid_b, io_ref) != 0:
                raise RuntimeError("bind failed")

    exec_fn, inst = m.dl.nxt_model_instance_exec, m.instance
    one_args = [(one[4], one[3]) for one in singles]

    def sync_step():
        # the reference scheduler's pattern: one instance_exec(.., 1) per
        # request (scheduler.c:477-488), each synchronous.  (The loop calls
        # the C entry point with prebuilt arguments: the reference's
        # scheduler is C, and Python's per-call overhead, ~0.5 us, is not
        # part of the pattern.)
        for ptr, n in one_args:
            rc = exec_fn(inst, ptr, n)
            if rc != 0:
                return rc
        return 0

    def deferred_step():
        # the same calls in deferred mode, then one flush
        for ptr, n in one_args:
            rc = exec_fn(inst, ptr, n)
            if rc != 0:
                return rc
        return m.flush()

    # One exec over the whole batch per step; with --per-request the deferred
    # mode takes turns with it step by step (both see the same batch), and
    # then as many steps run synchronously, one exec per request, on their
    # own: so each is timed in its steady state (a one-request exec right
    # after a batched exec of the same sequence first uploads that
    # sequence's device record; in a scheduler's loop of one-request execs
    # the records stay current).  Every step appends a token per request, so
    # the synchronous steps attend over somewhat longer contexts.
    blocks = [[("whole", lambda: m.exec_requests(batch))]]
    if args.per_request:
        blocks[0].append(("deferred", deferred_step))
        blocks.append([("synchronous", sync_step)])
    timed = {key: [] for block in blocks for key, _ in block}
    for block in blocks:
        for step in range(args.warmup + args.steps):
            for key, fn in block:
                if key == "deferred":
                    assert m.set_deferred(True) == 0
                bind_step()
                t0 = time.perf_counter()
                rc = fn()
                dt = time.perf_counter() - t0
                if key == "deferred":
                    assert m.set_deferred(False) == 0
                if rc != 0:
                    raise RuntimeError(f"{key} exec failed at step {step}")
                if step >= args.warmup:
                    timed[key].append(dt)
    times = timed["whole"]
    # the whole-batch execs attend over the prompt lengths plus (modes taking
    # turns) x (steps so far) + 1 tokens; the middle one:
    turns = len(blocks[0])
    mid_lens = lens + turns * (args.warmup + args.steps // 2) + 1
    per_request = None
    if args.per_request:
        per_request = {}
        for key in ("synchronous", "deferred"):
            t = timed[key]
            md = float(np.median(t))
            mode_mid = (lens + 2 * (args.warmup + args.steps) + args.warmup + args.steps // 2 + 1
                        if key == "synchronous" else mid_lens + 1)
            per_request[key] = {"seqs_per_s": round(nreq / md, 1),
                                "step_us": {"median": round(md * 1e6, 1),
                                            "min": round(min(t) * 1e6, 1),
                                            "max": round(max(t) * 1e6, 1)},
                                "context_tokens_at_timed_middle": int(mode_mid.sum())}
        log(f"[bench] per-request execs: {per_request}")
    ok = bool(torch.isfinite(out.float()).all())
    exec_count = int(m.model.instances[0].exec_count)
    med = float(np.median(times))
    m.close()
    del m
    torch.cuda.empty_cache()
    # The same batch's bare attention step (one nxt_paged_attention call over
    # a synthetic batch of the timed execs' middle lengths; plain-decode
    # configs), and the launch floor of a synchronous exec on this runtime.
    # (Config 5's batch shares pages through the index, which a synthetic
    # batch of the same lengths would not: no bare step there.)
    bare = None
    rng_b = np.random.default_rng(11)
    if args.config != 5:
        wl_mid = W._make(f"{name}-serve-mid", 11, mid_lens, H=H, KVH=KVH, D=D, bs=bs,
                         kv_dtype=kv_dtype, pool_factor=1, rng=rng_b, poison=False)
        bare = {"step_us": round(bare_decode_step_us(wl_mid, 200, 200), 1),
                "context_tokens": int(mid_lens.sum())}
        log(f"[bench] bare attention step over the timed execs' middle lengths: {bare}")
    wl1 = W._make(f"{name}-one-request", 12, [int(np.round(mid_lens.mean()))], H=H, KVH=KVH,
                  D=D, bs=bs, kv_dtype=kv_dtype, pool_factor=1, rng=rng_b, poison=False)
    floor = launch_floor(wl1)
    log(f"[bench] launch floor (host-timed from Python): {floor}")
    log(f"[bench] serve {name}: {nreq} requests, prefill {t_prefill:.2f} s; decode exec median "
        f"{med * 1e6:.1f} us (min {min(times) * 1e6:.1f}, max {max(times) * 1e6:.1f}); "
        f"finite outputs: {ok}")
    if per_request:
        per_request["deferred_over_whole_batch"] = round(
            per_request["deferred"]["step_us"]["median"] / (med * 1e6), 3)
        per_request["synchronous_over_whole_batch"] = round(
            per_request["synchronous"]["step_us"]["median"] / (med * 1e6), 3)
    print(json.dumps({
        "metric": "decode step through the model instance (instance_exec, whole batch)",
        "value": round(nreq / med, 1), "unit": "seqs/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(med * 1e3, 4), "higher_is_better": True,
        "dtype": {W.FP16: "fp16", W.BF16: "bf16", W.FP32: "fp32"}[kv_dtype],
        "data": "synthetic (seeded prompts of the config's lengths, random K/V on device)",
        "config": {"workload": name, "requests": nreq, "context_tokens": int(lens.sum())},
        "exec_us": {"median": round(med * 1e6, 1), "min": round(min(times) * 1e6, 1),
                    "max": round(max(times) * 1e6, 1)},
        "instance_exec_count": exec_count,
        "context_tokens_at_timed_middle": int(mid_lens.sum()),
        **({"bare_step_same_lengths": bare} if bare else {}),
        **({"exec_over_bare_step": round(med * 1e6 / bare["step_us"], 3)} if bare else {}),
        **({"launch_floor": floor} if floor else {}),
        **({"per_request": per_request} if per_request else {}),
        "check": {"outputs_finite": ok}}), flush=True)
    return 0 if ok else 1


def _pct(xs, q):
    import numpy as np
    return round(float(np.percentile(np.asarray(xs, dtype=np.float64), q)), 2) if len(xs) else None


def wg_trace_report(args, wl, lib, step, i0, stream, ms_per_step, alg_bytes, entry, waves) -> int:
    """Per-workgroup timeline of one step through the instrumented build
    (xllms_amd/csrc/wg_trace.h): 5 traced steps, the last one summarised.
    Times in us from the first workgroup's entry (s_memrealtime, 100 MHz)."""
    import numpy as np
    import torch
    words = int(lib.xhip_wg_trace_words())
    buf = torch.zeros(words, dtype=torch.int64, device="cuda")
    for i in range(5):
        buf.zero_()
        torch.cuda.synchronize()
        lib.xhip_set_wg_trace(buf.data_ptr())
        step(i0 + i)
        lib.xhip_set_wg_trace(None)
        torch.cuda.synchronize()
    rec = buf.cpu().numpy().view(np.uint64).astype(np.int64)
    np.save(args.wg_trace + ".npy", rec)  # the raw words, for further reading
    W_ = 24  # words per partition record (xllms_amd/csrc/wg_trace.h)
    part = rec[:4096 * W_].reshape(4096, W_)
    used = part[:, 0] > 0
    part = part[used]
    merge = rec[4096 * W_:].reshape(-1, 2)
    merge = merge[merge[:, 0] > 0]
    t0 = int(part[:, 0].min())
    us = lambda x: (np.asarray(x, dtype=np.int64) - t0) / 100.0  # noqa: E731
    info = part[:, 3]
    role = (info >> 32) & 0xFF
    entry_us, exit_us = us(part[:, 0]), us(part[:, 2])
    groups = np.nonzero(used)[0]
    # the segment kernel stamps wavefront 0's first and last tile in [7], [8]
    # and has no prologue stamp; the MFMA kernels stamp every wavefront
    segment = not (part[:, 4] > 0).any() and bool((part[:, 7] > 0).any())
    lines = []
    lines.append(f"# Per-workgroup timeline: {wl.name}" + (" (cascade)" if args.cascade else ""))
    lines.append("")
    argv = list(sys.argv[1:])
    for i, a in enumerate(argv):  # the output path stands as <out>.md
        if a == "--wg-trace" and i + 1 < len(argv):
            argv[i + 1] = "<out>.md"
        elif a.startswith("--wg-trace="):
            argv[i] = "--wg-trace=<out>.md"
    lines.append(f"Command: `python bench.py {' '.join(argv)}`")
    lines.append("")
    lines.append(f"Instrumented build `libxllm_hip_backend_trace.so` (XHIP_WG_TRACE, "
                 f"`xllms_amd/csrc/wg_trace.h`): s_memrealtime stamps (100 MHz) per workgroup "
                 f"of one step, the 5th of 5 traced steps after {args.warmup} warm-up and "
                 f"{2 * args.steps} untraced steps. Times in us from the first workgroup's entry. "
                 f"Untraced step in the same run: {ms_per_step * 1e3:.2f} us.")
    lines.append("")
    roles = {0: "all", 1: "prefix body", 2: "suffix body"}
    summary = {"workload": wl.name, "cascade": bool(args.cascade), "step_us": round(ms_per_step * 1e3, 2),
               "workgroups": int(used.sum()), "merge_workgroups": int(len(merge))}
    lines.append("| Workgroups | n | entry p50 / max | prologue done p50 / p90 / max | "
                 "first tile p50 / max | last tile done p10 / p50 / p90 / max | exit p10 / p50 / p90 / max |")
    lines.append("|---|---|---|---|---|---|---|")
    for r in sorted(set(role.tolist())):
        sel = role == r
        if segment:
            ft, le = part[sel][:, 7], part[sel][:, 8]
        else:
            wf = part[sel][:, 4:16].reshape(-1, 4, 3)
            ft = wf[:, :, 0].ravel()
            le = wf[:, :, 1].ravel()
        ft_us, le_us = us(ft[ft > 0]), us(le[le > 0])
        pro = part[sel][:, 1]
        pro_us = us(pro[pro > 0])
        row = {"n": int(sel.sum()),
               "entry": [_pct(entry_us[sel], 50), _pct(entry_us[sel], 100)],
               "prologue_done": [_pct(pro_us, q) for q in (50, 90, 100)],
               "first_tile": [_pct(ft_us, 50), _pct(ft_us, 100)],
               "last_tile_done": [_pct(le_us, q) for q in (10, 50, 90, 100)],
               "exit": [_pct(exit_us[sel], q) for q in (10, 50, 90, 100)]}
        summary[roles.get(r, str(r))] = row
        lines.append(f"| {roles.get(r, str(r))} | {row['n']} | {row['entry'][0]} / {row['entry'][1]} | "
                     f"{' / '.join(map(str, row['prologue_done'])) if row['prologue_done'][0] is not None else 'n/a'} | "
                     f"{row['first_tile'][0]} / {row['first_tile'][1]} | "
                     f"{' / '.join(map(str, row['last_tile_done']))} | "
                     f"{' / '.join(map(str, row['exit']))} |")
    extra = [w for w in range(16, W_) if (part[:, w] > 0).mean() > 0.5]
    if extra:
        lines.append("")
        lines.append("Kernel-specific phase stamps (`wg_trace.h`), p50 / max: " + ", ".join(
            f"[{w}] {_pct(us(part[:, w][part[:, w] > 0]), 50)} / "
            f"{_pct(us(part[:, w][part[:, w] > 0]), 100)}" for w in extra))
    # per XCD (dispatch deals workgroup b to XCD b % 8)
    xcd = groups % 8
    lines.append("")
    lines.append("Exit by XCD (workgroup b runs on XCD b % 8), p50 / max: " + ", ".join(
        f"{x}: {_pct(exit_us[xcd == x], 50)} / {_pct(exit_us[xcd == x], 100)}" for x in range(8)))
    if segment:
        lines.append("")
        lines.append("Segment kernel (one workgroup per segment or share of one): first tile and "
                     "last tile done are wavefront 0's; no prologue stamp (no split-unit scan).")
    else:
        # streaming rate per wavefront: tiles x bytes per tile / (last tile done - first tile)
        tile_bytes = 16 * wl.head_size * wl.elem_bytes * 2
        wf = part[:, 4:16].reshape(-1, 4, 3).reshape(-1, 3)
        ok = (wf[:, 0] > 0) & (wf[:, 1] > wf[:, 0])
        tiles = wf[ok, 2] & 0xFFFFFFFF
        pieces = wf[ok, 2] >> 32
        dur = (wf[ok, 1] - wf[ok, 0]) / 100.0
        rate = tiles * tile_bytes / np.maximum(dur, 1e-3) / 1e3  # GB/s
        lines.append("")
        lines.append(f"Wavefronts with tiles: {int(ok.sum())}; tiles per wavefront p10 / p50 / max "
                     f"{_pct(tiles, 10)} / {_pct(tiles, 50)} / {_pct(tiles, 100)}; pieces p50 / max "
                     f"{_pct(pieces, 50)} / {_pct(pieces, 100)}; per-wavefront K/V rate (first tile "
                     f"issued to last tile done) p10 / p50 / p90 {_pct(rate, 10)} / {_pct(rate, 50)} / "
                     f"{_pct(rate, 90)} GB/s.")
        summary["tiles_per_wave"] = [_pct(tiles, 10), _pct(tiles, 50), _pct(tiles, 100)]
        summary["wave_rate_gbs"] = [_pct(rate, 10), _pct(rate, 50), _pct(rate, 90)]
    if len(merge):
        me, mx = us(merge[:, 0]), us(merge[:, 1][merge[:, 1] > 0])
        summary["merge"] = {"entry": [_pct(me, 0), _pct(me, 50), _pct(me, 100)],
                            "exit": [_pct(mx, 50), _pct(mx, 100)]}
        lines.append("")
        lines.append(f"Merge launch: {len(merge)} workgroups; entry min / p50 / max "
                     f"{_pct(me, 0)} / {_pct(me, 50)} / {_pct(me, 100)}; exit p50 / max "
                     f"{_pct(mx, 50)} / {_pct(mx, 100)}.")
    span = float(exit_us.max())
    summary["partition_span_us"] = round(span, 2)
    lines.append("")
    lines.append(f"Partition launch span (first entry to last exit): {span:.2f} us; algorithmic "
                 f"bytes {alg_bytes} = {alg_bytes / (span * 1e-6) / 1e9:.0f} GB/s over it.")
    text = "\n".join(lines) + "\n"
    with open(args.wg_trace, "w") as f:
        f.write(text)
    log(text)
    print(json.dumps({"metric": "per-workgroup timeline (instrumented build)", **summary}), flush=True)
    return 0


SHAPE_FLAGS = ("batch", "ctx", "heads", "kv_heads", "head_size", "dtype", "block_size")


def workload_from_args(args):
    """--config's workload, or the reference bench's shape when any of its
    flags is given (defaults tests/test_attention_bench.c:34-41)."""
    from xllms_amd import workloads as W
    if all(getattr(args, f) is None for f in SHAPE_FLAGS):
        return W.make(args.config)
    if args.cascade:
        raise SystemExit("--cascade needs a shared-prefix --config, not the reference-bench shape")
    dt = {"fp16": W.FP16, "bf16": W.BF16, "fp32": W.FP32}[args.dtype or "fp16"]
    return W.ref_bench_shape(batch=args.batch or 16, ctx=args.ctx or 1024, heads=args.heads or 32,
                             kv_heads=args.kv_heads or 8, head_size=args.head_size or 128,
                             kv_dtype=dt, block_size=args.block_size or 16)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", "--iterations", dest="steps", type=int, default=200,
                    help="timed steps (--iterations: the reference bench's name for it)")
    ap.add_argument("--warmup", type=int, default=200,
                    help="untimed steps first (>= ~20 ms of work: the GPU clocks ramp up over it)")
    ap.add_argument("--config", type=int, default=2, help="1..5, 6 = config 4b (GQA16)")
    # The reference bench's shape flags (tests/test_attention_bench.c:421-435; its
    # defaults :34-41).  Any of them selects that workload instead of --config:
    # every sequence at --ctx tokens, seeded N(0,1) data, a permuted table.
    ap.add_argument("--batch", type=int, default=None, help="reference-bench shape: sequences (16)")
    ap.add_argument("--ctx", type=int, default=None, help="reference-bench shape: context (1024)")
    ap.add_argument("--heads", type=int, default=None, help="reference-bench shape: q heads (32)")
    ap.add_argument("--kv-heads", type=int, default=None,
                    help="reference-bench shape: kv heads (8)")
    ap.add_argument("--head-size", type=int, default=None,
                    help="reference-bench shape: head size (128)")
    ap.add_argument("--dtype", choices=["fp16", "bf16", "fp32"], default=None,
                    help="reference-bench shape: K/V element type (fp16)")
    ap.add_argument("--block-size", type=int, default=None,
                    help="reference-bench shape: tokens per page (16)")
    ap.add_argument("--partition", type=int, default=0,
                    help="split-K tokens per wavefront (0 = automatic stream-K plan)")
    ap.add_argument("--pools", type=int, default=0, help="K/V pool copies to rotate (0 = auto)")
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-check", action="store_true", help="skip the post-run oracle check")
    ap.add_argument("--cascade", action="store_true",
                    help="prefix-aware decode (nxt_paged_attention_cascade): shared prefixes found "
                         "once from the block tables (nxt_paged_prefix_groups, outside the timed "
                         "steps), each step one cascade call")
    ap.add_argument("--serve", action="store_true",
                    help="decode steps through the plugin's model instance (configs 2, 4, 5, 6)")
    ap.add_argument("--per-request", action="store_true",
                    help="with --serve: also time the reference scheduler's pattern, one "
                         "instance_exec(.., 1) per request per step, synchronous and in deferred "
                         "mode (queued, one flush per step)")
    ap.add_argument("--kv-append", action="store_true",
                    help="instead of the attention, time the KV append on the workload's shape: "
                         "every token of the batch written through nxt_paged_kv_write_slots "
                         "(HBM-bound) and one decode step through nxt_paged_kv_append")
    ap.add_argument("--activation", choices=sorted(ACT_OPS), default=None,
                    help="instead of the attention, time this MLP activation (reference entry "
                         "point, fp16, Llama-3-8B intermediate size 14336) over --act-tokens")
    ap.add_argument("--act-tokens", type=int, default=8192)
    ap.add_argument("--copy-peak", action="store_true",
                    help="instead of the benchmark, measure the ceilings the roofline fraction "
                         "is read against: a plain 1 GiB device copy and the workload's K/V "
                         "access pattern streamed with no arithmetic (xllm_stream_probe)")
    ap.add_argument("--wg-trace", default=None, metavar="MD",
                    help="after the timed steps, run 5 steps through the instrumented build "
                         "(libxllm_hip_backend_trace.so) and write the per-workgroup timeline "
                         "of the last to MD (markdown); the JSON line is then that summary")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="instead of the benchmark, run 5 plain device copies of MIB MiB "
                         "(the reference kernel for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the paged-decode path is sharded by sequence or kv head with no exchange, so the "
              "per-GPU figure is the one to report", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    if args.copy_calibration:
        n = args.copy_calibration * 2**20 // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": n * 4, "copy_calibration_bytes_written": n * 4,
                          "copies": 5}))
        return 0

    from xllms_amd import paged_attention as PA
    from xllms_amd import workloads as W

    if args.serve:
        return bench_serve(args)
    if args.kv_append:
        return bench_kv_append(args)
    if args.activation:
        return bench_activation(args)

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    dev = torch.device("cuda:0")

    t0 = time.perf_counter()
    wl = workload_from_args(args)
    log(f"[bench] workload {wl.name}: {wl.describe()} built in {time.perf_counter() - t0:.1f}s")
    alg_bytes = wl.algorithmic_bytes()
    logical_bytes = wl.logical_bytes()

    dw = W.upload(wl, dev)
    pool_bytes = 2 * dw.key_cache.numel() * dw.key_cache.element_size()
    pools = args.pools or max(3, -(-768 * 2**20 // pool_bytes))
    kpools, vpools = [dw.key_cache], [dw.value_cache]
    for _ in range(pools - 1):
        kpools.append(dw.key_cache.clone())
        vpools.append(dw.value_cache.clone())
    torch.cuda.synchronize()
    log(f"[bench] {pools} K/V pools of {pool_bytes / 2**20:.0f} MiB each resident in HBM")

    stream = torch.cuda.current_stream().cuda_stream
    lib = PA._lib.backend(trace=bool(args.wg_trace))
    entry = "nxt_paged_attention" if args.partition == 0 and wl.kv_dtype != W.BF16 else None
    waves = PA.auto_waves(wl.num_seqs, wl.num_heads, wl.head_size, wl.num_kv_heads,
                          wl.max_num_blocks_per_seq, wl.block_size, wl.kv_dtype)

    if args.copy_peak:
        probe = pattern_peak(wl, kpools, vpools, waves, args.steps, distinct=args.cascade)
        copy = device_copy_peak()
        log(f"[bench] access-pattern probe {probe}; device copy {copy}")
        print(json.dumps({"workload": wl.name, "hbm_spec_gbs": HBM_PEAK_GBS,
                          "pattern_read": probe, "device_copy": copy,
                          "note": "pattern_read: this batch's K/V tiles streamed with the "
                                  "decode kernel's loads (16-byte nontemporal, one tile in "
                                  "flight, same wavefront count) and no arithmetic; "
                                  "device_copy: read + write bytes of a 1 GiB copy"}),
              flush=True)
        return 0

    # Pre-marshalled arguments: the timed loop is one ctypes call per step.
    fn = getattr(lib, entry) if entry else lib.nxt_paged_attention_ex
    def args_for(kc, vc):
        a = (dw.out.data_ptr(), dw.query.data_ptr(), kc.data_ptr(), vc.data_ptr(),
             dw.block_tables.data_ptr(), dw.seq_lens.data_ptr(), wl.num_seqs, wl.num_heads,
             wl.head_size, wl.num_kv_heads, ctypes.c_float(wl.scale), wl.max_num_blocks_per_seq,
             wl.block_size, wl.elem_bytes, wl.kv_block_stride, wl.kv_head_stride, stream)
        return a if entry else a + (wl.kv_dtype, args.partition)
    n_groups = None
    if args.cascade:
        # once per batch composition, as a server would: find the shared prefixes
        pgroup, pblocks, pcount = PA.prefix_groups(dw.block_tables, dw.seq_lens,
                                                   block_size=wl.block_size)
        torch.cuda.synchronize()
        n_groups = int(pcount.cpu()[0])
        entry = "nxt_paged_attention_cascade"
        fn = lib.nxt_paged_attention_cascade
        def args_for(kc, vc):  # noqa: F811
            return (dw.out.data_ptr(), dw.query.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                    dw.block_tables.data_ptr(), dw.seq_lens.data_ptr(), pgroup.data_ptr(),
                    pblocks.data_ptr(), max(n_groups, 0), wl.num_seqs, wl.num_heads,
                    wl.head_size, wl.num_kv_heads, ctypes.c_float(wl.scale),
                    wl.max_num_blocks_per_seq, wl.block_size, wl.kv_block_stride,
                    wl.kv_head_stride, wl.kv_dtype, stream)
        log(f"[bench] cascade: {n_groups} shared-prefix groups found")
    call_args = [args_for(k, v) for k, v in zip(kpools, vpools)]

    def step(i: int) -> None:
        fn(*call_args[i % pools])

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    st, msg = PA.last_status()
    if st != 0:
        raise RuntimeError(f"launch failed: {msg}")

    # The K timed steps: back-to-back calls bracketed by two events.
    ev = HipEvents()
    begin, end = ev.create(), ev.create()
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    ev.record(begin, stream)
    for i in range(args.steps):
        step(args.warmup + i)
    ev.record(end, stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    st, msg = PA.last_status()
    if st != 0:
        raise RuntimeError(f"launch failed: {msg}")
    total_ms = ev.elapsed_ms(begin, end)
    # The partition kernel's launch durations: K more steps of the same
    # calls, the library stamping two events with each partition kernel's
    # start and end (hipExtLaunchKernel, on the stream it runs on).  Kept out
    # of the timed steps, which carry no instrumentation.
    if args.cascade:
        kern_ms = np.array([total_ms / args.steps])
    else:
        k_start = [ev.create() for _ in range(args.steps)]
        k_done = [ev.create() for _ in range(args.steps)]
        for i in range(args.steps):
            lib.nxt_attn_set_trace_events(k_start[i], k_done[i])
            step(args.warmup + args.steps + i)
        lib.nxt_attn_set_trace_events(None, None)
        torch.cuda.synchronize()
        st, msg = PA.last_status()
        if st != 0:
            raise RuntimeError(f"launch failed: {msg}")
        kern_ms = np.array([ev.elapsed_ms(a, b) for a, b in zip(k_start, k_done)])
    ev.destroy_all()

    if args.wg_trace:
        return wg_trace_report(args, wl, lib, step, args.warmup + 2 * args.steps, stream,
                               total_ms / args.steps, alg_bytes, entry, waves)

    ms_per_step = total_ms / args.steps
    # A cascade step is several kernels (plan, two partition + merge passes,
    # combine): its roofline figure uses the whole step.
    kernel_avg_ms = ms_per_step if args.cascade else float(kern_ms.mean())
    value = wl.num_seqs / (ms_per_step / 1e3)
    achieved = alg_bytes / (kernel_avg_ms / 1e3) / 1e9
    log(f"[bench] {args.steps} steps: {ms_per_step * 1e3:.1f} us/step (wall {wall / args.steps * 1e6:.1f}"
        f" us), {'cascade step' if args.cascade else 'partition kernel'} "
        f"{kernel_avg_ms * 1e3:.1f} us avg "
        f"(min {kern_ms.min() * 1e3:.1f}, max {kern_ms.max() * 1e3:.1f}), "
        f"{achieved:.0f} GB/s = {achieved / HBM_PEAK_GBS:.1%} of 8 TB/s, "
        f"step {alg_bytes / (ms_per_step / 1e3) / 1e9:.0f} GB/s")

    check = None
    if not args.no_check:
        from oracle import oracle as O
        from tests.helpers import assert_close
        got = dw.out.float().cpu().numpy()
        idx = np.arange(0, wl.num_seqs, max(1, wl.num_seqs // 8))
        ref = O.run_workload(wl, precision="mt", seqs=idx)
        stats = assert_close(got[idx], ref, wl.kv_dtype, "bench output")
        check = {"seqs_checked": int(len(idx)), **stats}
        log(f"[bench] output matches the oracle on {len(idx)} sequences: {stats}")

    cpu = None
    if not args.no_cpu_baseline:
        c = cpu_baseline(wl, args.cpu_budget)
        tok_per_seq = wl.tokens() / wl.num_seqs
        cpu = {"value": round(c["all"]["seqs_per_s"], 2), "unit": "seqs/s",
               "cores": c["all"]["threads"], "kind": "port",
               "sample": (f"oracle/paged_attention_oracle.c (C restatement of text_gen.c:1284-1310"
                          f" over the operator-API buffers, gcc -O2, OpenMP over (seq, head)) on "
                          f"{c['all']['seqs']} sequences of this batch ({c['all']['tokens']} "
                          f"context tokens) in {c['all']['seconds']:.1f}s; seqs/s by tokens over "
                          f"the batch's tokens per sequence"),
               "single_thread": {"value": round(c["single"]["seqs_per_s"], 3), "cores": 1,
                                 "sample": f"{c['single']['seqs']} sequences "
                                           f"({c['single']['tokens']} tokens) in "
                                           f"{c['single']['seconds']:.1f}s"},
               "gbs_all_threads": round(c["all"]["seqs_per_s"] * alg_bytes / wl.num_seqs / 1e9, 2),
               "tokens_per_seq": round(tok_per_seq, 1)}
        log(f"[bench] cpu baseline: {cpu}")

    # The ceilings the kernel is read against, measured in this run: the
    # batch's own K/V access pattern with no arithmetic, and a plain copy.
    probe = pattern_peak(wl, kpools, vpools, waves, 50, distinct=args.cascade)
    copy = device_copy_peak()
    step_gbs = alg_bytes / (ms_per_step / 1e3) / 1e9
    measured_peak = {
        "pattern_read_gbs": probe["gbs"] if probe else None,
        "pattern_read": ("the batch's compulsory K/V tiles" if args.cascade else
                         "the batch's K/V tiles") + " streamed with the decode kernel's loads and "
                         "wavefront count, no arithmetic (xllm_stream_probe)",
        "device_copy_gbs": copy["gbs"],
        # time ratios: the probe streams the same tiles the kernel reads
        "kernel_frac_of_pattern": round(probe["us"] / (kernel_avg_ms * 1e3), 4) if probe else None,
        "step_frac_of_pattern": round(probe["us"] / (ms_per_step * 1e3), 4) if probe else None,
    }
    log(f"[bench] measured ceilings: {measured_peak}")

    traffic = load_traffic(wl.name + ("_cascade" if args.cascade else ""))
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "seqs/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {W.FP16: "fp16", W.BF16: "bf16", W.FP32: "fp32"}[wl.kv_dtype],
        "data": "synthetic (seeded N(0,1) Q/K/V, seeded ragged lengths and page tables)",
        "config": {"workload": wl.name, "num_seqs": wl.num_seqs, "num_heads": wl.num_heads,
                   "num_kv_heads": wl.num_kv_heads, "head_size": wl.head_size,
                   "block_size": wl.block_size, "tokens": wl.tokens(),
                   "context_range": [int(wl.seq_lens.min()), int(wl.seq_lens.max())],
                   "split_k": ("stream-K, %d wavefronts" % waves) if args.partition == 0
                   else f"{args.partition} tokens per wavefront", "kv_pools_rotated": pools,
                   "entry_point": entry or "nxt_paged_attention_ex", "seed": wl.seed,
                   **({"prefix_groups": n_groups} if args.cascade else {})},
        "achieved_gbs_step": round(alg_bytes / (ms_per_step / 1e3) / 1e9, 1),
        "algorithmic_bytes": alg_bytes,
        "logical_bytes": logical_bytes,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "step_frac": round(step_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "kernel": ("cascade decode step (one partition launch that plans and "
                                "computes the prefix and suffix batches, merge)") if args.cascade
                     else partition_kernel_name(wl),
                     "kernel_avg_us": round(kernel_avg_ms * 1e3, 2)},
        "measured_peak": measured_peak,
        "cpu_baseline": cpu,
        "check": check,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
