"""Seeded synthetic paged-decode workloads (the five benchmark configurations).

Every workload is host (numpy) buffers in the reference operator-API layout
(include/operator_api.h:45-60, strides as tests/test_attention.c:141-143):
  query            [B][H][D]                 element type
  key/value_cache  [num_blocks][KVH][bs][D]  element type
  block_tables     int32 [B][max_blocks], -1 past each sequence
  seq_lens         int32 [B]
16-bit data are stored as uint16 bit patterns (fp16 or bf16).

Randomness: lengths, pools and page permutations come from
numpy.random.default_rng(seed); Q/K/V values come from the counter-based
generator of libxllm_workload.so (element i of tensor stream t is a pure
function of (seed*16 + t, i)), so buffers are identical across machines and
thread counts.  seed = 20260000 + config number.

Garbage (configs 2-5): pages of the pool that no sequence references keep
random values with NaN / +Inf / -Inf sentinels written over them, and the K/V
slots past each sequence's end in its last page are NaN.  A correct kernel
never reads either.
"""
from __future__ import annotations

import ctypes
import dataclasses
import math

import numpy as np

from . import _lib

FP16, BF16, FP32 = 1, 2, 3
_ELEM_BYTES = {FP16: 2, BF16: 2, FP32: 4}
_NAN = {FP16: 0x7E00, BF16: 0x7FC0}
_PINF = {FP16: 0x7C00, BF16: 0x7F80}
_NINF = {FP16: 0xFC00, BF16: 0xFF80}
TAG_Q, TAG_K, TAG_V = 1, 2, 3


@dataclasses.dataclass
class Workload:
    name: str
    seed: int
    num_heads: int
    num_kv_heads: int
    head_size: int
    block_size: int
    kv_dtype: int
    scale: float
    seq_lens: np.ndarray
    block_tables: np.ndarray
    query: np.ndarray
    key_cache: np.ndarray
    value_cache: np.ndarray
    notes: str = ""

    @property
    def num_seqs(self) -> int:
        return int(self.seq_lens.shape[0])

    @property
    def num_blocks(self) -> int:
        return int(self.key_cache.shape[0])

    @property
    def max_num_blocks_per_seq(self) -> int:
        return int(self.block_tables.shape[1])

    @property
    def elem_bytes(self) -> int:
        return _ELEM_BYTES[self.kv_dtype]

    @property
    def kv_block_stride(self) -> int:
        return self.num_kv_heads * self.block_size * self.head_size

    @property
    def kv_head_stride(self) -> int:
        return self.block_size * self.head_size

    @property
    def group(self) -> int:
        return self.num_heads // self.num_kv_heads

    def tokens(self) -> int:
        return int(self.seq_lens.clip(min=0).sum())

    def referenced_blocks(self) -> int:
        return int(sum(-(-int(L) // self.block_size) for L in self.seq_lens if L > 0))

    def distinct_page_tokens(self) -> int:
        """Sum over distinct physical pages of the valid tokens they hold."""
        fill: dict[int, int] = {}
        bs = self.block_size
        for s, L in enumerate(self.seq_lens):
            L = int(L)
            for j in range(-(-L // bs)):
                blk = int(self.block_tables[s, j])
                n = min(bs, L - j * bs)
                if n > fill.get(blk, 0):
                    fill[blk] = n
        return sum(fill.values())

    def _extra_bytes(self) -> int:
        e = self.elem_bytes
        return (2 * self.num_seqs * self.num_heads * self.head_size * e   # Q and O
                + 4 * self.referenced_blocks() + 4 * self.num_seqs)      # tables, lengths

    def algorithmic_bytes(self) -> int:
        """Compulsory HBM traffic of one launch: distinct K/V rows once, Q, O,
        the referenced block-table entries and seq_lens."""
        kv = self.distinct_page_tokens() * self.num_kv_heads * 2 * self.head_size * self.elem_bytes
        return kv + self._extra_bytes()

    def logical_bytes(self) -> int:
        """Bytes if every sequence streamed its own K/V (no prefix sharing)."""
        kv = self.tokens() * self.num_kv_heads * 2 * self.head_size * self.elem_bytes
        return kv + self._extra_bytes()

    def flops(self) -> int:
        return 4 * self.head_size * self.num_heads * self.tokens()

    def describe(self) -> dict:
        return {
            "workload": self.name, "seed": self.seed, "num_seqs": self.num_seqs,
            "num_heads": self.num_heads, "num_kv_heads": self.num_kv_heads,
            "head_size": self.head_size, "block_size": self.block_size,
            "kv_dtype": {FP16: "fp16", BF16: "bf16", FP32: "fp32"}[self.kv_dtype],
            "tokens": self.tokens(), "num_blocks": self.num_blocks,
            "max_num_blocks_per_seq": self.max_num_blocks_per_seq,
            "context_min": int(self.seq_lens.min()), "context_max": int(self.seq_lens.max()),
        }


def _np_dtype(kv_dtype: int):
    return np.float32 if kv_dtype == FP32 else np.uint16


def fill_normal(arr: np.ndarray, kv_dtype: int, stream_seed: int, offset: int = 0,
                mul: float = 1.0, threads: int = 0) -> None:
    assert arr.flags.c_contiguous and arr.dtype == _np_dtype(kv_dtype)
    _lib.workload().xw_fill_normal(arr.ctypes.data, arr.size, kv_dtype, stream_seed, offset,
                                   ctypes.c_float(mul), threads)


def normal_values(n: int, stream_seed: int, offset: int = 0, kv_dtype: int = FP32) -> np.ndarray:
    out = np.empty(n, dtype=_np_dtype(kv_dtype))
    fill_normal(out, kv_dtype, stream_seed, offset)
    return out


def _tables_for(seq_lens: np.ndarray, block_size: int, pool_pages: np.ndarray,
                max_blocks: int) -> np.ndarray:
    """Give each sequence its pages, in logical order, from pool_pages."""
    tables = np.full((len(seq_lens), max_blocks), -1, dtype=np.int32)
    pos = 0
    for s, L in enumerate(seq_lens):
        n = -(-int(L) // block_size)
        tables[s, :n] = pool_pages[pos:pos + n]
        pos += n
    return tables


def _fill_kv(wl: Workload, threads: int = 0) -> None:
    fill_normal(wl.key_cache, wl.kv_dtype, wl.seed * 16 + TAG_K, threads=threads)
    fill_normal(wl.value_cache, wl.kv_dtype, wl.seed * 16 + TAG_V, threads=threads)


def _poison(wl: Workload) -> None:
    """NaN/Inf sentinels in unreferenced pages, NaN in the tail slots."""
    if wl.kv_dtype == FP32:
        nan, pinf, ninf = np.float32(np.nan), np.float32(np.inf), np.float32(-np.inf)
    else:
        nan, pinf, ninf = (np.uint16(_NAN[wl.kv_dtype]), np.uint16(_PINF[wl.kv_dtype]),
                           np.uint16(_NINF[wl.kv_dtype]))
    used = np.zeros(wl.num_blocks, dtype=bool)
    bs = wl.block_size
    for s, L in enumerate(wl.seq_lens):
        n = -(-int(L) // bs)
        used[wl.block_tables[s, :n]] = True
    unused = np.nonzero(~used)[0]
    for cache in (wl.key_cache, wl.value_cache):
        flat = cache.reshape(cache.shape[0], -1)
        for i in range(0, len(unused), 4096):
            idx = unused[i:i + 4096]
            sub = flat[idx]
            sub[:, ::7] = nan
            sub[:, 3::11] = pinf
            sub[:, 5::13] = ninf
            flat[idx] = sub
    for s, L in enumerate(wl.seq_lens):
        L = int(L)
        if L <= 0 or L % bs == 0:
            continue
        last = int(wl.block_tables[s, (L - 1) // bs])
        wl.key_cache[last, :, L % bs:, :] = nan
        wl.value_cache[last, :, L % bs:, :] = nan


def _make(name, seed, seq_lens, *, H, KVH, D, bs, kv_dtype, pool_factor, rng, poison,
          tables=None, num_blocks=None, notes="") -> Workload:
    seq_lens = np.asarray(seq_lens, dtype=np.int32)
    need = int(sum(-(-int(L) // bs) for L in seq_lens))
    max_blocks = max(1, int(max(-(-int(L) // bs) for L in seq_lens)))
    if tables is None:
        num_blocks = max(1, need * pool_factor)
        pages = rng.permutation(num_blocks)[:need].astype(np.int32)
        tables = _tables_for(seq_lens, bs, pages, max_blocks)
    B = len(seq_lens)
    dt = _np_dtype(kv_dtype)
    wl = Workload(name=name, seed=seed, num_heads=H, num_kv_heads=KVH, head_size=D,
                  block_size=bs, kv_dtype=kv_dtype, scale=1.0 / math.sqrt(D),
                  seq_lens=seq_lens, block_tables=tables,
                  query=np.empty((B, H, D), dtype=dt),
                  key_cache=np.empty((num_blocks, KVH, bs, D), dtype=dt),
                  value_cache=np.empty((num_blocks, KVH, bs, D), dtype=dt), notes=notes)
    fill_normal(wl.query, kv_dtype, seed * 16 + TAG_Q)
    _fill_kv(wl)
    if poison:
        _poison(wl)
    return wl


def config1(seed: int = 20260001, num_seqs: int = 8) -> Workload:
    """GPT-2-small shape, fp32, MHA: 12/12 heads, d=64, bs=16, L ~ U{16..1024};
    pool = exactly the pages needed, randomly permuted."""
    rng = np.random.default_rng(seed)
    L = rng.integers(16, 1024, size=num_seqs, endpoint=True)
    return _make("gpt2-small-mha-fp32", seed, L, H=12, KVH=12, D=64, bs=16, kv_dtype=FP32,
                 pool_factor=1, rng=rng, poison=False)


def config2(seed: int = 20260002, num_seqs: int = 64, lo: int = 512, hi: int = 4096) -> Workload:
    """Llama-3-8B GQA shape (headline): 32 q / 8 kv heads, d=128, fp16, bs=16,
    L ~ U{512..4096}; pool = 2x the pages needed, the rest garbage."""
    rng = np.random.default_rng(seed)
    L = rng.integers(lo, hi, size=num_seqs, endpoint=True)
    return _make("llama3-8b-gqa4-fp16", seed, L, H=32, KVH=8, D=128, bs=16, kv_dtype=FP16,
                 pool_factor=2, rng=rng, poison=True)


def config3(seed: int = 20260003, lens=(8192, 16384, 24576, 32768),
            spike_frac: float = 0.01, spike_mul: float = 8.0) -> Workload:
    """Long-context split-K stress: Llama-3-8B heads, fp16, L = 8k/16k/24k/32k;
    1% of the valid (seq, token, kv-head) K rows scaled by 8 before rounding."""
    rng = np.random.default_rng(seed)
    wl = _make("long-context-splitk-fp16", seed, list(lens), H=32, KVH=8, D=128, bs=16,
               kv_dtype=FP16, pool_factor=2, rng=rng, poison=False)
    rows = []
    bs, KVH = wl.block_size, wl.num_kv_heads
    for s, Ls in enumerate(wl.seq_lens):
        Ls = int(Ls)
        n = max(1, int(round(spike_frac * Ls * KVH)))
        pick = rng.choice(Ls * KVH, size=n, replace=False)
        tok, kvh = pick // KVH, pick % KVH
        blk = wl.block_tables[s, tok // bs].astype(np.int64)
        rows.append((blk * KVH + kvh) * bs + tok % bs)
    rows = np.sort(np.concatenate(rows)).astype(np.int64)
    _lib.workload().xw_scale_rows(wl.key_cache.ctypes.data, rows.ctypes.data, rows.size,
                                  wl.head_size, wl.kv_dtype, wl.seed * 16 + TAG_K, 0,
                                  ctypes.c_float(spike_mul), 0)
    _poison(wl)
    wl.notes = f"{rows.size} spiked K rows x{spike_mul}"
    return wl


def config4(seed: int = 20260004, num_kv_heads: int = 8, num_seqs: int = 128) -> Workload:
    """70B shape: 64 q heads, 8 kv heads (G8) or 4 (G16), d=128, bf16, bs=16,
    L = clip(round(exp(N(ln 1024, 0.8))), 1, 8192); pool 2x, rest garbage."""
    rng = np.random.default_rng(seed)
    L = np.clip(np.round(np.exp(rng.normal(math.log(1024.0), 0.8, size=num_seqs))), 1, 8192)
    name = f"llama-70b-gqa{64 // num_kv_heads}-bf16"
    return _make(name, seed, L.astype(np.int64), H=64, KVH=num_kv_heads, D=128, bs=16,
                 kv_dtype=BF16, pool_factor=2, rng=rng, poison=True)


def config5(seed: int = 20260005, num_seqs: int = 256, groups: int = 16,
            fresh_frac: float = 0.10) -> Workload:
    """Continuous batching with radix-shared prefixes: 32/8 heads, d=128, fp16,
    bs=16, B=256.  10% of sequences have L=1; the rest fall round-robin into 16
    groups whose members share the physical pages of a common prefix of
    P ~ U{256..2048} tokens (floor(P/16) full pages; the P mod 16 remainder
    is copied into each member's first private page), then a private suffix
    S ~ U{1..1024}."""
    rng = np.random.default_rng(seed)
    bs, KVH, D = 16, 8, 128
    n_fresh = int(math.floor(fresh_frac * num_seqs))
    prefix = rng.integers(256, 2048, size=groups, endpoint=True)
    seq_group = np.full(num_seqs, -1, dtype=np.int64)
    seq_group[n_fresh:] = np.arange(num_seqs - n_fresh) % groups
    suffix = rng.integers(1, 1024, size=num_seqs, endpoint=True)
    L = np.where(seq_group < 0, 1, prefix[np.maximum(seq_group, 0)] + suffix).astype(np.int64)
    shared_blocks = prefix // bs
    n_shared = int(shared_blocks.sum())
    private = [(-(-int(L[s]) // bs)) - (int(shared_blocks[seq_group[s]]) if seq_group[s] >= 0 else 0)
               for s in range(num_seqs)]
    need = n_shared + int(sum(private))
    num_blocks = 2 * need
    pages = rng.permutation(num_blocks)[:need].astype(np.int32)
    max_blocks = int(max(-(-int(x) // bs) for x in L))
    tables = np.full((num_seqs, max_blocks), -1, dtype=np.int32)
    group_pages, pos = [], 0
    for g in range(groups):
        group_pages.append(pages[pos:pos + int(shared_blocks[g])])
        pos += int(shared_blocks[g])
    for s in range(num_seqs):
        g = int(seq_group[s])
        k = 0
        if g >= 0:
            tables[s, :len(group_pages[g])] = group_pages[g]
            k = len(group_pages[g])
        tables[s, k:k + private[s]] = pages[pos:pos + private[s]]
        pos += private[s]
    wl = _make("radix-shared-prefix-fp16", seed, L, H=32, KVH=KVH, D=D, bs=bs, kv_dtype=FP16,
               pool_factor=2, rng=rng, poison=False, tables=tables, num_blocks=num_blocks)
    # The prefix remainder (P mod 16 tokens) is a copy of the same prefix
    # tokens in every member: take the first member's rows as the template.
    for g in range(groups):
        rem = int(prefix[g]) % bs
        members = np.nonzero(seq_group == g)[0]
        if rem == 0 or len(members) == 0:
            continue
        k = int(shared_blocks[g])
        src = int(tables[members[0], k])
        for s in members[1:]:
            dst = int(tables[s, k])
            wl.key_cache[dst, :, :rem, :] = wl.key_cache[src, :, :rem, :]
            wl.value_cache[dst, :, :rem, :] = wl.value_cache[src, :, :rem, :]
    _poison(wl)
    wl.notes = f"{n_fresh} fresh (L=1) sequences, {groups} prefix groups"
    return wl


def ref_bench_shape(batch: int = 16, ctx: int = 1024, heads: int = 32, kv_heads: int = 8,
                    head_size: int = 128, kv_dtype: int = FP16, block_size: int = 16,
                    seed: int = 20260010) -> Workload:
    """The reference bench's workload shape (tests/test_attention_bench.c:34-41
    defaults: batch 16, context 1024, 32 q / 8 kv heads, d 128, fp16, block
    size 16; every sequence at the full context, :134-137): a pool of exactly
    the pages the batch needs.  Unlike the reference's buffers (zeros and an
    identity block table, :125-139), Q/K/V are seeded N(0,1) and the table is
    a seeded permutation of the pool, so the output check means something."""
    if min(batch, ctx, heads, kv_heads, head_size, block_size) <= 0 or heads % kv_heads:
        raise ValueError("batch, ctx, heads, kv_heads, head_size, block_size must be positive "
                         "and heads a multiple of kv_heads")
    rng = np.random.default_rng(seed)
    name = (f"refbench-b{batch}-ctx{ctx}-{heads}x{kv_heads}-d{head_size}-"
            f"{ {FP16: 'fp16', BF16: 'bf16', FP32: 'fp32'}[kv_dtype] }")
    return _make(name, seed, [ctx] * batch, H=heads, KVH=kv_heads, D=head_size, bs=block_size,
                 kv_dtype=kv_dtype, pool_factor=1, rng=rng, poison=True)


def serve_prompts(config: int, token_seed: int = 7):
    """Token-level prompts with the sequence lengths of a config's batch (the
    same seeded draws as its generator) for the serving path, which builds
    its own K/V; no K/V pool is made here.  Config 5 keeps its sharing: each
    group's members start with the same P-token prefix.  Returns
    (workload name, num_heads, num_kv_heads, head_size, kv_dtype, prompts)."""
    tok = np.random.default_rng(token_seed)
    if config == 5:
        rng = np.random.default_rng(20260005)
        B, groups, n_fresh = 256, 16, 25
        prefix = rng.integers(256, 2048, size=groups, endpoint=True)
        suffix = rng.integers(1, 1024, size=B, endpoint=True)
        heads = [tok.integers(0, 32000, int(p)).astype(np.int32) for p in prefix]
        prompts = [tok.integers(0, 32000, 1).astype(np.int32) for _ in range(n_fresh)]
        for s in range(n_fresh, B):
            g = (s - n_fresh) % groups
            prompts.append(np.concatenate([heads[g], tok.integers(0, 32000, int(suffix[s]))
                                           .astype(np.int32)]))
        return "radix-shared-prefix-fp16", 32, 8, 128, FP16, prompts
    if config == 2:
        rng = np.random.default_rng(20260002)
        L = rng.integers(512, 4096, size=64, endpoint=True)
        name, H, KVH, D, dt = "llama3-8b-gqa4-fp16", 32, 8, 128, FP16
    elif config in (4, 6):
        rng = np.random.default_rng(20260004)
        L = np.clip(np.round(np.exp(rng.normal(math.log(1024.0), 0.8, size=128))), 1, 8192)
        KVH = 8 if config == 4 else 4
        name, H, D, dt = f"llama-70b-gqa{64 // KVH}-bf16", 64, 128, BF16
    else:
        raise ValueError(f"serving prompts are defined for configs 2, 4, 5, 6, not {config}")
    return name, H, KVH, D, dt, [tok.integers(0, 32000, int(n)).astype(np.int32) for n in L]


CONFIGS = {
    1: config1,
    2: config2,
    3: config3,
    4: config4,
    5: config5,
}


def make(config: int, **kw) -> Workload:
    if config == 6:  # 4b: GQA16
        return config4(num_kv_heads=4, **kw)
    return CONFIGS[config](**kw)


def small_case(*, num_seqs=3, H=8, KVH=2, D=128, bs=16, kv_dtype=FP16, lens=None, seed=7,
               pool_factor=2, poison=True, max_len=200) -> Workload:
    """Small randomized case for the parity tests (seconds on the CPU checker)."""
    rng = np.random.default_rng(seed)
    if lens is None:
        lens = rng.integers(1, max_len, size=num_seqs, endpoint=True)
    lens = [int(x) for x in lens]
    if max(lens) <= 0:
        raise ValueError("need at least one non-empty sequence")
    seq_lens = np.asarray(lens, dtype=np.int32)
    need = int(sum(-(-max(L, 0) // bs) for L in lens))
    max_blocks = max(1, max(-(-max(L, 0) // bs) for L in lens))
    num_blocks = max(1, need * pool_factor)
    pages = rng.permutation(num_blocks)[:need].astype(np.int32)
    tables = np.full((len(lens), max_blocks), -1, dtype=np.int32)
    pos = 0
    for s, L in enumerate(lens):
        n = -(-max(L, 0) // bs)
        tables[s, :n] = pages[pos:pos + n]
        pos += n
    wl = _make(f"small-{H}x{KVH}-d{D}-bs{bs}", seed, seq_lens, H=H, KVH=KVH, D=D, bs=bs,
               kv_dtype=kv_dtype, pool_factor=pool_factor, rng=rng, poison=False, tables=tables,
               num_blocks=num_blocks)
    if poison:
        _poison(wl)
    return wl


def torch_dtype(kv_dtype: int):
    import torch
    return {FP16: torch.float16, BF16: torch.bfloat16, FP32: torch.float32}[kv_dtype]


def to_torch(arr: np.ndarray, kv_dtype: int, device="cuda"):
    """Host element bits -> torch tensor of the element type on `device`."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(arr))
    if kv_dtype != FP32:
        t = t.view(torch.int16)
    return t.to(device).view(torch_dtype(kv_dtype))


@dataclasses.dataclass
class DeviceWorkload:
    query: object
    key_cache: object
    value_cache: object
    block_tables: object
    seq_lens: object
    out: object


def upload(wl: Workload, device="cuda") -> DeviceWorkload:
    import torch
    return DeviceWorkload(
        query=to_torch(wl.query, wl.kv_dtype, device),
        key_cache=to_torch(wl.key_cache, wl.kv_dtype, device),
        value_cache=to_torch(wl.value_cache, wl.kv_dtype, device),
        block_tables=torch.from_numpy(np.ascontiguousarray(wl.block_tables)).to(device),
        seq_lens=torch.from_numpy(np.ascontiguousarray(wl.seq_lens)).to(device),
        out=torch.full(wl.query.shape, float("nan"), dtype=torch_dtype(wl.kv_dtype),
                       device=device),
    )
