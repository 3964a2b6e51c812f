#!/usr/bin/env python3
"""Benchmark of the paged KV-cache hot path on one MI355X.

A step is one decode step of one layer over a batch of sequences: the KV
append of one new token per sequence and paged decode attention over every
sequence's whole context, in one fused call (skv_paged_decode_append; with
--separate: skv_kv_append then skv_paged_decode).  Inputs are synthetic and
already resident in HBM when timing starts; the step rewrites each sequence's
last slot (context stays the same from step to step, as the reference's
forward_into with append_tokens=false does), so every timed step does
identical work.  Config 5 adds the churn work of its definition before the
decode step (block-table rows of the 4 new sequences, their 2,048-token
prefill chunks appended through the tables).

Default workload: config 4 of BASELINE.json (Llama-3-8B geometry: 32 Q heads,
8 KV heads, head_dim 128, batch 128, context lengths log-normal with median
8192 and sigma 0.6 clipped to [2048, 32768], 16-token blocks allocated
round-robin across sequences), the configuration the >= 70 % of HBM peak
target is quoted on.  --config 2 / 3 / 5 select the other single-GPU
attention configs; --config 1 times the same call per layer and position of
a 22-layer TinyLlama-shaped generation (16 prompt + 128 new tokens).

Output: one JSON line on stdout.  value = algorithmic bytes of a whole step
/ device time per step, in GB/s.  roofline = the decode call (fused append +
attention kernel, then the merge kernel) against 8 TB/s.  cpu_baseline = the
oracle's restatement of the reference CPU attention timed on this host on a
bounded sample of sequences of the same workload.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "paged decode-attn achieved HBM GB/s (% of peak) + decode tokens/sec, 1 GPU"
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, AMD public specification
# Table sets cycled through by the timed steps of configs whose step reads less
# than a few times the 256 MB last-level cache (cfg3: 8 x 285 MB).
CACHE_ROTATION = 8


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# Workloads
# ---------------------------------------------------------------------------
def lifo_round_robin_tables(nbs, max_blocks):
    """Tables as a fresh BlockPool hands blocks out (0, 1, 2, ...) when the
    sequences take one block each in turn (round-robin, fragmented pool)."""
    t = np.full((len(nbs), max_blocks), -1, np.int32)
    nxt = 0
    for k in range(max(nbs)):
        for b, nb in enumerate(nbs):
            if k < nb:
                t[b, k] = nxt
                nxt += 1
    return t, nxt


def workload(cfg: int):
    bs = 16
    if cfg == 2:
        rng = np.random.default_rng(0x5EED0002)
        Hq, Hkv, hd, B = 32, 4, 64, 1
        lens = np.array([4097], np.int32)            # 4096 cached + the appended token
        total = 65536
        perm = rng.permutation(total).astype(np.int32)
        nb = -(-4097 // bs)
        tables = perm[:nb].reshape(1, nb)
        # Timed steps cycle through disjoint tables (consecutive 257-id slices of
        # the same permutation), so no step re-reads what the step before left
        # in the 256 MB last-level cache.
        rotation = [perm[i * nb:(i + 1) * nb].reshape(1, nb) for i in range(total // nb)]
        desc = ("cfg2: batch 1, 32 Q / 4 KV heads, head_dim 64, context 4097 (4096 + 1 appended), "
                "table = first 257 ids of a seeded permutation of a 65536-block pool; timed steps "
                "cycle through the permutation's 255 disjoint 257-id tables")
    elif cfg == 3:
        rng = np.random.default_rng(0x5EED0003)
        Hq, Hkv, hd, B = 32, 4, 64, 64
        lens = rng.integers(512, 8193, size=B).astype(np.int32)
        total = 1 << 20
        perm = rng.permutation(total).astype(np.int32)
        nbs = [-(-int(L) // bs) for L in lens]
        rotation = []
        pos = 0
        for _ in range(CACHE_ROTATION):
            t = np.full((B, max(nbs)), -1, np.int32)
            for b, nb in enumerate(nbs):
                t[b, :nb] = perm[pos:pos + nb]
                pos += nb
            rotation.append(t)
        tables = rotation[0]
        desc = ("cfg3: batch 64, TinyLlama geometry (32 Q / 4 KV heads, head_dim 64), contexts "
                "U[512, 8192], tables = consecutive slices of a seeded permutation of a 2^20-block pool; "
                f"timed steps cycle through {CACHE_ROTATION} disjoint table sets (the next slices)")
    elif cfg == 4:
        rng = np.random.default_rng(0x5EED0004)
        Hq, Hkv, hd, B = 32, 8, 128, 128
        z = rng.standard_normal(B)
        lens = np.clip(np.round(np.exp(math.log(8192) + 0.6 * z)), 2048, 32768).astype(np.int32)
        nbs = [-(-int(L) // bs) for L in lens]
        tables, used = lifo_round_robin_tables(nbs, max(nbs))
        total = used + 1024
        desc = ("cfg4: Llama-3-8B geometry (32 Q / 8 KV heads, head_dim 128), batch 128, contexts "
                "log-normal median 8192 sigma 0.6 clipped to [2048, 32768], 16-token blocks "
                "allocated round-robin across sequences")
    elif cfg == 5:
        return churn_workload()
    else:
        raise SystemExit(f"bench.py: unknown --config {cfg} (configs: 1, 2, 3, 4, 5)")
    w = dict(cfg=cfg, Hq=Hq, Hkv=Hkv, hd=hd, B=B, bs=bs, lens=lens, tables=tables,
             total=int(total), desc=desc, seed=0x5EED0000 + cfg)
    if cfg in (2, 3):
        w["rotation"] = rotation
    return w


def contiguous_tables(w):
    """The same workload with each sequence's blocks consecutive, in a pool of
    exactly the blocks the tables use (sequence 0's first, then sequence 1's,
    ...): the block order that reads the least scattered memory, to measure
    what a config's own block placement costs the load pattern."""
    nbs = [int(np.count_nonzero(row >= 0)) for row in w["tables"]]
    tables = np.full_like(w["tables"], -1)
    pos = 0
    for b, nb in enumerate(nbs):
        tables[b, :nb] = np.arange(pos, pos + nb, dtype=np.int32)
        pos += nb
    w = dict(w, tables=tables, total=int(pos),
             desc=w["desc"] + "; tables replaced by consecutive ids in a pool of the blocks used")
    w.pop("rotation", None)
    return w


class LifoPool:
    """Block ids in BlockPool order: the constructor's stack holds total-1 ... 0
    (block 0 on top) and freed ids are pushed in table order, so the last block
    of a freed sequence is handed out first (src/memory/block_pool.cpp:72-76,
    193-207; src/memory/page_table.cpp:152-160)."""

    def __init__(self, total: int):
        self.stack = list(range(total - 1, -1, -1))

    def alloc(self) -> int:
        if not self.stack:
            raise RuntimeError("OOM")
        return self.stack.pop()

    def free(self, ids) -> None:
        self.stack.extend(ids)


CHURN_LONG, CHURN_NEW, CHURN_L, CHURN_CHUNK = 32, 4, 131072, 2048


def churn_workload(steps: int = 64):
    """cfg5: 64 Q / 8 KV heads, head_dim 128.  32 sequences of 131,072 tokens
    (blocks allocated round-robin) plus 4 churn slots.  Before the first step
    4 further long sequences are evicted, so their 4 x 8,192 blocks sit on top
    of the free stack.  Step s: free the 4 churn sequences of step s-1, allocate
    4 new ones and chunk-append one 2,048-token prefill chunk to each (128
    blocks each, taken LIFO, i.e. freed blocks in reverse: non-monotone
    tables), append one decode token to all 36 sequences, decode all 36.
    Returns the table state for every step (precomputed on the host)."""
    bs, Hq, Hkv, hd = 16, 64, 8, 128
    nbl = CHURN_L // bs
    n_live = CHURN_LONG + CHURN_NEW
    total = (CHURN_LONG + CHURN_NEW) * nbl + 64
    pool = LifoPool(total)
    long_tables = np.zeros((n_live, nbl), np.int32)
    for k in range(nbl):                      # 36 long sequences, round-robin
        for i in range(n_live):
            long_tables[i, k] = pool.alloc()
    for i in range(CHURN_LONG, n_live):       # evict 4 of them
        pool.free(long_tables[i].tolist())
    new_blocks = CHURN_CHUNK // bs + 1        # the chunk plus the decode token's block
    churn = np.zeros((steps, CHURN_NEW, new_blocks), np.int32)
    prev = None
    for st in range(steps):
        if prev is not None:
            for row in prev:
                pool.free(row.tolist())
        for j in range(CHURN_NEW):
            churn[st, j] = [pool.alloc() for _ in range(new_blocks)]
        prev = churn[st]
    tables = np.full((n_live, nbl), -1, np.int32)
    tables[:CHURN_LONG] = long_tables[:CHURN_LONG]
    tables[CHURN_LONG:, :new_blocks] = churn[0]
    lens = np.array([CHURN_L] * CHURN_LONG + [CHURN_CHUNK + 1] * CHURN_NEW, np.int32)
    desc = ("cfg5: 64 Q / 8 KV heads, head_dim 128; 32 sequences at 131,072 tokens + 4 churn slots; "
            "each step frees the previous 4 churn sequences, chunk-appends one 2,048-token prefill "
            "chunk to 4 new ones (LIFO-reused blocks, non-monotone tables), appends one decode token "
            "to all 36 and decodes all 36")
    return dict(cfg=5, Hq=Hq, Hkv=Hkv, hd=hd, B=n_live, bs=bs, lens=lens, tables=tables,
                total=int(total), desc=desc, seed=0x5EED0005, churn=churn)


def algorithmic_bytes(w):
    """Bytes each step must move at least once (K/V counted once per KV head).
    Returns (decode bytes, append bytes, flops); for cfg5 the append bytes
    include the 4 x 2,048-token chunk append and the table patch."""
    B, Hq, Hkv, hd, bs = w["B"], w["Hq"], w["Hkv"], w["hd"], w["bs"]
    L = w["lens"].astype(np.int64)
    kv = int((2 * L * Hkv * hd * 2).sum())
    tables = int((4 * np.ceil(L / bs)).sum()) + 4 * B
    qo = B * Hq * hd * 2 + B * Hq * hd * 4
    decode = kv + tables + qo
    token_append = B * 2 * Hkv * hd * 2 * 2
    churn_append = 0
    if "churn" in w:
        churn_append = CHURN_NEW * CHURN_CHUNK * 2 * Hkv * hd * 2 * 2 + 2 * 4 * w["churn"][0].size
    flops = 4 * int(L.sum()) * Hq * hd
    return decode, token_append, churn_append, flops


# ---------------------------------------------------------------------------
# GPU run
# ---------------------------------------------------------------------------
def setup_gpu(w):
    """The step's device inputs, resident in HBM: seeded N(0,1) bf16 pools,
    queries and new rows, the tables and lengths, the output and workspace."""
    import stratakv_amd as skv

    skv.require_gpu()
    B, Hq, Hkv, hd, bs, total = w["B"], w["Hq"], w["Hkv"], w["hd"], w["bs"], w["total"]
    pool_elems = total * bs * Hkv * hd
    log(f"allocating pools: 2 x {pool_elems * 2 / 2**30:.2f} GiB")
    d = dict(skv=skv, stream=skv.Stream())
    h = d["stream"].handle
    d["k_pool"] = skv.DeviceBuffer(pool_elems * 2)
    d["v_pool"] = skv.DeviceBuffer(pool_elems * 2)
    skv.fill_normal_bf16(d["k_pool"], pool_elems, w["seed"], 0, h)
    skv.fill_normal_bf16(d["v_pool"], pool_elems, w["seed"] + 1, 0, h)
    d["q"] = skv.DeviceBuffer(B * Hq * hd * 2)
    skv.fill_normal_bf16(d["q"], B * Hq * hd, w["seed"] + 2, 0, h)
    d["k_new"] = skv.DeviceBuffer(B * Hkv * hd * 2)
    d["v_new"] = skv.DeviceBuffer(B * Hkv * hd * 2)
    skv.fill_normal_bf16(d["k_new"], B * Hkv * hd, w["seed"] + 3, 0, h)
    skv.fill_normal_bf16(d["v_new"], B * Hkv * hd, w["seed"] + 4, 0, h)
    d["tables"] = skv.DeviceBuffer.from_numpy(w["tables"])
    # Per-step tables: the rotation's table sets one after another in one buffer.
    rot = w.get("rotation")
    if rot is not None:
        d["rot_buf"] = skv.DeviceBuffer.from_numpy(np.ascontiguousarray(np.stack(rot)))
        d["rot_ptrs"] = [d["rot_buf"].ptr + i * rot[0].nbytes for i in range(len(rot))]
    else:
        d["rot_ptrs"] = [d["tables"].ptr]
    d["lens"] = skv.DeviceBuffer.from_numpy(w["lens"])
    d["positions"] = skv.DeviceBuffer.from_numpy(w["lens"] - 1)
    d["out"] = skv.DeviceBuffer(B * Hq * hd * 4)
    d["ws"], d["wsb"] = skv.decode_workspace(B, Hq, Hkv, hd, h)
    d["max_blocks"] = w["tables"].shape[1]
    d["scale"] = 1.0 / math.sqrt(hd)
    d["stream"].synchronize()
    return d


def run_gpu(w, steps: int, warmup: int, fused: bool = True):
    """Times `steps` decode steps.  A step is [pre] + [main]: with fused=True,
    pre = the cfg5 churn work (table patch + prefill-chunk append; nothing for
    the other configs) and main = one skv_paged_decode_append call (decode-token
    append + attention); with fused=False, pre also holds the decode-token
    skv_kv_append and main is skv_paged_decode alone."""
    d = setup_gpu(w)
    skv, stream = d["skv"], d["stream"]
    B, Hq, Hkv, hd, bs, total = w["B"], w["Hq"], w["Hkv"], w["hd"], w["bs"], w["total"]
    k_pool, v_pool, q, k_new, v_new = d["k_pool"], d["v_pool"], d["q"], d["k_new"], d["v_new"]
    tables, lens, positions, out = d["tables"], d["lens"], d["positions"], d["out"]
    ws, wsb, max_blocks, scale = d["ws"], d["wsb"], d["max_blocks"], d["scale"]
    log("inputs resident; warming up")

    churn = w.get("churn")
    if churn is not None:
        assert churn.shape[0] >= warmup + 2 * steps, "churn history shorter than the run"
        churn_dev = skv.DeviceBuffer.from_numpy(churn)
        n_chunk = CHURN_NEW * CHURN_CHUNK * Hkv * hd
        chunk_k = skv.DeviceBuffer(n_chunk * 2)
        chunk_v = skv.DeviceBuffer(n_chunk * 2)
        skv.fill_normal_bf16(chunk_k, n_chunk, w["seed"] + 5, 0, stream.handle)
        skv.fill_normal_bf16(chunk_v, n_chunk, w["seed"] + 6, 0, stream.handle)
        zero_pos = skv.DeviceBuffer.from_numpy(np.zeros(CHURN_NEW, np.int32))
        row_bytes = churn.shape[2] * 4
        step_counter = [0]

    def pre():
        if churn is not None:
            # New churn sequences: their block-table rows, then the prefill chunk.
            st = step_counter[0]
            step_counter[0] += 1
            for j in range(CHURN_NEW):
                src = churn_dev.ptr + (st * CHURN_NEW + j) * row_bytes
                dst = tables.ptr + ((CHURN_LONG + j) * max_blocks) * 4
                skv._check(skv.lib().skv_memcpy_d2d(dst, src, row_bytes, stream.handle))
            skv.kv_append(chunk_k, chunk_v, skv.DTYPE_BF16, k_pool, v_pool, total,
                          tables.ptr + CHURN_LONG * max_blocks * 4, max_blocks, zero_pos,
                          CHURN_NEW, CHURN_CHUNK, Hkv, hd, bs, stream=stream.handle)
        if not fused:
            t = rot_ptrs[main_counter[0] % len(rot_ptrs)]
            skv.kv_append(k_new, v_new, skv.DTYPE_BF16, k_pool, v_pool, total, t, max_blocks,
                          positions, B, 1, Hkv, hd, bs, stream=stream.handle)

    rot_ptrs = d["rot_ptrs"]
    main_counter = [0]

    def main():
        t = rot_ptrs[main_counter[0] % len(rot_ptrs)]
        main_counter[0] += 1
        if fused:
            skv.paged_decode_append(q, skv.DTYPE_BF16, k_new, v_new, skv.DTYPE_BF16, k_pool, v_pool,
                                    total, t, max_blocks, lens, B, Hq, Hkv, hd, bs, scale, out,
                                    ws, wsb, stream=stream.handle)
        else:
            skv.paged_decode(q, skv.DTYPE_BF16, k_pool, v_pool, total, t, max_blocks, lens, B,
                             Hq, Hkv, hd, bs, scale, out, ws, wsb, stream=stream.handle)

    for _ in range(warmup):
        pre()
        main()
    skv.synchronize()
    log(f"warmup done ({warmup} steps); timing {steps} steps")

    # The timed region: `steps` steps back to back, one event on the launch
    # stream before the first and one after the last (per-step events would
    # themselves take time between the launches of short steps).
    e_first, e_last = skv.Event(), skv.Event()
    skv.synchronize()
    t0 = time.perf_counter()
    e_first.record(stream.handle)
    for _ in range(steps):
        pre()
        main()
    e_last.record(stream.handle)
    skv.synchronize()
    wall = time.perf_counter() - t0
    total_ms = e_first.elapsed_ms(e_last)
    log(f"timed: device {total_ms:.3f} ms, host wall {wall * 1e3:.3f} ms")

    # A second pass of `steps` steps for the breakdown, with events on the
    # launch stream per step i: a before pre, b between pre and main, c after
    # main (when pre is empty, a is b).
    has_pre = churn is not None or not fused
    ev_a = [skv.Event() for _ in range(steps)]
    ev_b = [skv.Event() for _ in range(steps)] if has_pre else ev_a
    ev_c = [skv.Event() for _ in range(steps)]
    for i in range(steps):
        ev_a[i].record(stream.handle)
        if has_pre:
            pre()
            ev_b[i].record(stream.handle)
        main()
        ev_c[i].record(stream.handle)
    skv.synchronize()
    pre_ms = [ev_a[i].elapsed_ms(ev_b[i]) if has_pre else 0.0 for i in range(steps)]
    main_ms = [ev_b[i].elapsed_ms(ev_c[i]) for i in range(steps)]
    return dict(ms_per_step=total_ms / steps, pre_ms=float(np.mean(pre_ms)),
                main_ms=float(np.mean(main_ms)), main_ms_median=float(np.median(main_ms)),
                main_ms_min=float(np.min(main_ms)), wall_ms_per_step=wall * 1e3 / steps)


def block_bytes(w):
    """K/V bytes of every block the decode reads (whole 16-row blocks)."""
    nb = np.minimum(-(-w["lens"].astype(np.int64) // w["bs"]), w["tables"].shape[1])
    return int(nb.sum()) * w["bs"] * w["Hkv"] * w["hd"] * 2 * 2


def run_load_calibration(w, steps: int, warmup: int, rounds: int = 5):
    """The decode's load pattern alone (skv_paged_block_checksum: the MFMA
    decode kernel's grid, block order and buffer loads, the math replaced by a
    checksum) timed beside the bench's decode call on the same inputs, in
    `rounds` interleaved rounds of `steps` launches each."""
    d = setup_gpu(w)
    skv, stream = d["skv"], d["stream"]
    h = stream.handle
    B, Hq, Hkv, hd, bs, total = w["B"], w["Hq"], w["Hkv"], w["hd"], w["bs"], w["total"]
    sums = skv.DeviceBuffer(B * Hkv * 4)

    def checksum():
        skv.paged_block_checksum(d["k_pool"], d["v_pool"], total, d["tables"], d["max_blocks"], d["lens"],
                                 B, Hq, Hkv, hd, bs, sums, stream=h)

    def decode():
        skv.paged_decode_append(d["q"], skv.DTYPE_BF16, d["k_new"], d["v_new"], skv.DTYPE_BF16,
                                d["k_pool"], d["v_pool"], total, d["tables"], d["max_blocks"], d["lens"],
                                B, Hq, Hkv, hd, bs, d["scale"], d["out"], d["ws"], d["wsb"], stream=h)

    def timed(fn):
        ev = [skv.Event() for _ in range(steps + 1)]
        ev[0].record(h)
        for i in range(steps):
            fn()
            ev[i + 1].record(h)
        skv.synchronize()
        return [ev[i].elapsed_ms(ev[i + 1]) for i in range(steps)]

    for _ in range(warmup):
        checksum()
        decode()
    skv.synchronize()
    t_sum, t_dec = [], []
    for r in range(rounds):
        t_sum += timed(checksum)
        t_dec += timed(decode)
        log(f"round {r}: checksum {np.mean(t_sum[-steps:]) * 1e3:.1f} us, "
            f"decode call {np.mean(t_dec[-steps:]) * 1e3:.1f} us")
    got = sums.download(np.uint32, (B * Hkv,))
    kvb = block_bytes(w)
    dec_bytes, tok_bytes, _, _ = algorithmic_bytes(w)
    cs_ms, dec_ms = float(np.mean(t_sum)), float(np.mean(t_dec))
    print(json.dumps({
        "load_calibration": w["desc"],
        "block_bytes": kvb,
        "checksum_us": round(cs_ms * 1e3, 2),
        "checksum_us_min": round(float(np.min(t_sum)) * 1e3, 2),
        "checksum_gbs": round(kvb / (cs_ms / 1e3) / 1e9, 1),
        "decode_call_us": round(dec_ms * 1e3, 2),
        "decode_call_us_min": round(float(np.min(t_dec)) * 1e3, 2),
        "decode_call_gbs_on_block_bytes": round(kvb / (dec_ms / 1e3) / 1e9, 1),
        "decode_call_gbs_algorithmic": round((dec_bytes + tok_bytes) / (dec_ms / 1e3) / 1e9, 1),
        "decode_frac_of_load_ceiling": round(cs_ms / dec_ms, 4),
        "launches_each": steps * rounds,
        "checksum_xor": int(np.bitwise_xor.reduce(got)),
    }), flush=True)
    return 0


# ---------------------------------------------------------------------------
# CPU baseline: the oracle (restatement of src/layers/attention.cpp:263-337)
# ---------------------------------------------------------------------------
def host_cpu():
    """(logical CPUs of the host, CPUs this process may run on, CPU model)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 1
    return os.cpu_count() or 1, usable, model


def cpu_threads_all() -> int:
    """Threads for the all-cores leg: every CPU this process may run on, but
    no more than OMP_NUM_THREADS when that is set (the GPU boxes set it to the
    CPU share of one GPU, which is smaller than what the host reports)."""
    _, usable, _ = host_cpu()
    try:
        cap = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        cap = 0
    return max(1, min(usable, cap) if cap > 0 else usable)


def cpu_sample_tables(w, chosen):
    """The chosen sequences' rows of the config's own tables, with the block ids
    renumbered by rank into a pool of just the blocks they use: the blocks
    keep the order and interleaving they have in the config's pool (cfg4's
    round-robin placement, cfg3's shuffled slices) without allocating the
    config's whole pool on the host."""
    rows = w["tables"][chosen]
    nbs = [-(-int(L) // w["bs"]) for L in w["lens"][chosen]]
    used = np.concatenate([rows[i, :nb] for i, nb in enumerate(nbs)])
    order = np.unique(used)
    tables = np.full((len(chosen), max(nbs)), -1, np.int32)
    for i, nb in enumerate(nbs):
        tables[i, :nb] = np.searchsorted(order, rows[i, :nb])
    return tables, len(order)


def cpu_baseline(w, budget_s: float = 12.0):
    """The oracle's fp32 decode loops (restatement of
    src/layers/attention.cpp:263-337) on this host over a seeded sample of the
    config's sequences sized to about `budget_s` seconds on one thread, then
    the same sample on every usable core."""
    import oracle

    rng = np.random.default_rng(w["seed"] + 99)
    B, Hq, Hkv, hd, bs = w["B"], w["Hq"], w["Hkv"], w["hd"], w["bs"]
    order = rng.permutation(B)
    # Values do not change the loop's time: tile a 4 Mi-element random bf16 block.
    base = oracle.f32_to_bf16(rng.standard_normal(1 << 22, dtype=np.float32))
    scale = 1.0 / math.sqrt(hd)

    def sample(chosen):
        chosen = sorted(chosen)
        tables, tot = cpu_sample_tables(w, chosen)
        kp = np.resize(base, (tot, bs, Hkv, hd))
        vp = np.resize(base[::-1], (tot, bs, Hkv, hd))
        q = oracle.bf16_to_f32(np.resize(base[1::2], (len(chosen), Hq, hd)))
        return chosen, tables, tot, kp, vp, q

    # The host's rate: one sequence on one thread (multiply-adds of q.k and P.V
    # per key, query head and dimension per second); then take sequences up to
    # ~budget_s of single-thread work.
    _, tb, _, kp, vp, q = sample([int(order[0])])
    t0 = time.perf_counter()
    oracle.paged_decode(q, kp, vp, tb, w["lens"][[int(order[0])]].astype(np.int32), Hkv, bs, scale, threads=1)
    rate = int(w["lens"][order[0]]) * Hq * hd * 2 / max(time.perf_counter() - t0, 1e-6)
    chosen, macs = [], 0
    for b in order:
        chosen.append(int(b))
        macs += int(w["lens"][b]) * Hq * hd * 2
        if macs >= rate * budget_s:
            break
    chosen, tables, tot, kp, vp, q = sample(chosen)
    lens = w["lens"][chosen].astype(np.int32)
    sample_bytes = int((2 * lens.astype(np.int64) * Hkv * hd * 2).sum())
    nproc, usable, model = host_cpu()
    results = {}
    threads_all = cpu_threads_all()
    for threads in sorted({1, threads_all}):
        t0 = time.perf_counter()
        oracle.paged_decode(q, kp, vp, tables, lens, Hkv, bs, scale, threads=threads)
        dt = time.perf_counter() - t0
        results[threads] = dt
        log(f"cpu baseline: {len(chosen)} sequences, {threads} thread(s): {dt:.2f} s")
    full_kv = int((2 * w["lens"].astype(np.int64) * Hkv * hd * 2).sum())
    out = {}
    for threads, dt in results.items():
        gbs = sample_bytes / dt / 1e9
        out[threads] = dict(value=round(gbs, 4), unit="GB/s", cores=threads, kind="port",
                            nproc=nproc, cpus_usable=usable, cpu_model=model,
                            tokens_per_s=round(B / (full_kv / (gbs * 1e9)), 6),
                            sample=(f"oracle two-pass fp32 attention (restatement of "
                                    f"src/layers/attention.cpp:263-337, gcc -O3 -mavx2 -mfma) over "
                                    f"{len(chosen)} of {B} sequences ({int(lens.sum())} tokens, "
                                    f"{sample_bytes / 1e6:.1f} MB of bf16 K/V) through their rows of "
                                    f"the config's own block tables (ids renumbered by rank into a "
                                    f"pool of the {tot} blocks they use) in {dt:.2f} s on {threads} "
                                    f"thread(s); GB/s on the same algorithmic bytes, tokens/s scaled "
                                    f"by bytes to the full batch; the reference itself caches FP32, "
                                    f"so its real traffic is twice these bytes"))
    return out[1], out[threads_all]


# ---------------------------------------------------------------------------
# cfg1: the hot path of a TinyLlama-shaped generation, per layer per position
# ---------------------------------------------------------------------------
CFG1_LAYERS, CFG1_PROMPT, CFG1_NEW, CFG1_POOL_BLOCKS = 22, 16, 128, 1024


def cfg1_bytes(Hq, Hkv, hd, bs, positions, layers):
    """Algorithmic bytes of one generation: per layer and position p (context
    p + 1) the K/V read once, the table, the fp32 query and output, and the
    fp32 new rows read + bf16 rows written."""
    total = 0
    for p in range(positions):
        L = p + 1
        total += 2 * L * Hkv * hd * 2 + 4 * (-(-L // bs)) + 4 + Hq * hd * 4 * 2 + 2 * Hkv * hd * (4 + 2)
    return total * layers


def run_cfg1(steps: int, warmup: int, with_cpu: bool):
    """cfg1 of BASELINE.json on the GPU side: a TinyLlama-shaped model (32 Q / 4
    KV heads, head_dim 64, 22 layers, a 1,024-block pool per layer as the
    reference CLI sizes it) generating 16 prompt + 128 new tokens one position
    at a time, as forward_into runs them.  One step = one generation: for every
    position p and layer, one skv_paged_attention_decode_append call (the
    append of the token's fp32 K/V rows at p, then attention over p + 1 tokens,
    with the fp32 query) on that layer's pool -- the call forward_into makes.
    The GEMVs, norms and RoPE around it are not part of the measured path."""
    import stratakv_amd as skv

    skv.require_gpu()
    Hq, Hkv, hd, bs, layers = 32, 4, 64, 16, CFG1_LAYERS
    P = CFG1_PROMPT + CFG1_NEW
    rng = np.random.default_rng(0x5EED0001)
    q = skv.DeviceBuffer.from_numpy(rng.standard_normal((layers, P, Hq, hd), dtype=np.float32))
    kr = skv.DeviceBuffer.from_numpy(rng.standard_normal((layers, P, Hkv, hd), dtype=np.float32))
    vr = skv.DeviceBuffer.from_numpy(rng.standard_normal((layers, P, Hkv, hd), dtype=np.float32))
    pool_elems = CFG1_POOL_BLOCKS * bs * Hkv * hd
    kp = [skv.DeviceBuffer(pool_elems * 2) for _ in range(layers)]
    vp = [skv.DeviceBuffer(pool_elems * 2) for _ in range(layers)]
    for i in range(layers):
        skv.fill_normal_bf16(kp[i], pool_elems, 0x5EED0100 + 2 * i)
        skv.fill_normal_bf16(vp[i], pool_elems, 0x5EED0101 + 2 * i)
    # A fresh LIFO pool hands the one sequence blocks 0, 1, 2, ... in every layer.
    table = skv.DeviceBuffer.from_numpy(np.arange(-(-P // bs), dtype=np.int32))
    out = skv.DeviceBuffer(Hq * hd * 4)
    stream = skv.Stream()
    ws, wsb = skv.single_decode_workspace(Hq, Hkv, hd, stream.handle)
    scale = 1.0 / math.sqrt(hd)
    qrow, kvrow = Hq * hd * 4, Hkv * hd * 4

    def generation():
        for p in range(P):
            for i in range(layers):
                off = i * P + p
                skv.paged_attention_decode_append(
                    q.ptr + off * qrow, kr.ptr + off * kvrow, vr.ptr + off * kvrow, skv.DTYPE_FP32,
                    kp[i], vp[i], CFG1_POOL_BLOCKS, table, out, p + 1, bs, Hq, Hkv, hd, scale, ws,
                    wsb, stream=stream.handle)

    skv.synchronize()
    for _ in range(warmup):
        generation()
    skv.synchronize()
    log(f"cfg1 warmup done ({warmup} generations); timing {steps}")
    e0, e1 = skv.Event(), skv.Event()
    t0 = time.perf_counter()
    e0.record(stream.handle)
    for _ in range(steps):
        generation()
    e1.record(stream.handle)
    skv.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1) / steps
    nbytes = cfg1_bytes(Hq, Hkv, hd, bs, P, layers)
    calls = P * layers
    gbs = nbytes / (ms / 1e3) / 1e9
    line = {
        "metric": METRIC, "value": round(gbs, 3), "unit": "GB/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) fp32 queries and K/V rows, bf16 pools)",
        "config": {"workload": ("cfg1: TinyLlama-shaped generation, 22 layers x (16 prompt + 128 new) "
                                "positions, one skv_paged_attention_decode_append per layer and "
                                "position (32 Q / 4 KV heads, head_dim 64, 1,024-block pool per "
                                "layer); a step is one whole generation"),
                   "layers": layers, "positions": P, "num_q_heads": Hq, "num_kv_heads": Hkv,
                   "head_dim": hd, "block_size": bs, "parallelism": "none (1 GPU)"},
        "tokens_per_s": round(P / (ms / 1e3), 1),
        "us_per_layer_position": round(ms * 1e3 / calls, 3),
        "host_wall_ms_per_step": round(wall * 1e3 / steps, 3),
        "roofline": {"bound": "hbm", "note": "launch-bound: each call moves 20-90 KB",
                     "kernel": "skv_paged_attention_decode_append (fused append + attention, merge)",
                     "achieved": round(gbs, 3), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 6),
                     "traffic": profile_traffic("cfg1"),
                     "traffic_per": "generation (the sum over its 3,168 decode launches)",
                     "algorithmic_bytes": nbytes},
    }
    # The whole layer stack through the C++ API (TransformerBlock::forward_into
    # of every layer per token), when the driver is built.
    driver = os.path.join(ROOT, "build", "bin", "bench_layer_stack")
    if os.path.exists(driver):
        import subprocess
        proc = subprocess.run([driver, str(layers), str(P), "1"], stdout=subprocess.PIPE,
                              stderr=subprocess.PIPE, text=True, timeout=600)
        if proc.returncode == 0:
            stack = json.loads(proc.stdout.strip().splitlines()[-1])
            line["layer_stack"] = dict(stack, note=(
                "end-to-end forward_into of 22 TinyLlama-shaped layers per token (bf16 N(0,0.02) "
                "weights, GEMVs, norms, RoPE, fused append + decode, SwiGLU, residuals); "
                "embedding, lm_head and token choice are outside this measurement (the "
                "generator entry times them)"))
        else:
            log(f"layer stack driver failed ({proc.returncode}): {proc.stderr.strip()[-300:]}")
    # The whole generation through Generator::generate (embedding, 22 layers,
    # final norm, lm_head, greedy choice on the device), the reference CLI's run.
    gen_driver = os.path.join(ROOT, "build", "bin", "bench_generate")
    if os.path.exists(gen_driver):
        import subprocess
        proc = subprocess.run([gen_driver, "--repeat", "5"], stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                              text=True, timeout=600)
        if proc.returncode == 0:
            g = json.loads(proc.stdout.strip().splitlines()[-1])
            weight_bytes = 2 * (CFG1_LAYERS * (2 * 2048 * 2048 + 2 * 256 * 2048 + 3 * 5632 * 2048) + 32000 * 2048)
            g["weight_gbs_per_decode_token"] = round(weight_bytes / (g["decode_ms_per_token"] / 1e3) / 1e9, 1)
            line["generator"] = dict(g, note=(
                "Generator::generate of a TinyLlama-shaped model, bf16 N(0,0.02) weights, 16 prompt + 128 greedy "
                "tokens, everything on the device; tokens_per_s = 128 / gen time incl. the prompt (the "
                "reference CLI's pure_decode_tps definition); decode_ms_per_token from generate(128) - "
                "generate(1); weight_gbs = bf16 weight bytes read per decode token / decode time"))
        else:
            log(f"generate driver failed ({proc.returncode}): {proc.stderr.strip()[-300:]}")
        # A long prompt: the prompt pass (prefill_into of 2,048 tokens in one
        # chunk, projections as library GEMMs) and the first token.
        proc = subprocess.run([gen_driver, "--prompt", "2048", "--new", "1", "--repeat", "3"], stdout=subprocess.PIPE,
                              stderr=subprocess.PIPE, text=True, timeout=600)
        if proc.returncode == 0:
            g = json.loads(proc.stdout.strip().splitlines()[-1])
            ms = g["prefill_and_first_token_ms"]
            line["prompt_2048"] = {
                "ms": ms, "prompt_tokens_per_s": round(2048 / (ms / 1e3), 1),
                "first_call_ms": g.get("first_call_ms"),
                "unseen_2047_first_ms": g.get("unseen_length_first_ms"),
                "unseen_2047_second_ms": g.get("unseen_length_second_ms"),
                "note": ("Generator::generate(prompt of 2,048 ids, 1 new token): embedding, prefill_into of 22 "
                         "TinyLlama-shaped layers (q/k/v, o, gate/up, down as hipBLASLt bf16 GEMMs over the inputs "
                         "split into bf16 hi + lo, causal prefill attention), lm_head and the first greedy token; "
                         "first_call_ms: the process's first such call (opens the GEMM library, creates the "
                         "hipBLASLt handle, asks its heuristic for each shape); unseen_2047_*: a 2,047-token "
                         "prompt never run before, its first call (new GEMM shapes) and its second")}
        else:
            log(f"long-prompt driver failed ({proc.returncode}): {proc.stderr.strip()[-300:]}")
    if with_cpu:
        import oracle
        # One layer's 144 single-sequence decodes with the oracle, scaled to 22 layers.
        kpool = oracle.f32_to_bf16(rng.standard_normal((-(-P // bs), bs, Hkv, hd), dtype=np.float32))
        vpool = oracle.f32_to_bf16(rng.standard_normal((-(-P // bs), bs, Hkv, hd), dtype=np.float32))
        qh = rng.standard_normal((1, Hq, hd), dtype=np.float32)
        tab = np.arange(-(-P // bs), dtype=np.int32)[None, :]
        t0 = time.perf_counter()
        for p in range(P):
            oracle.paged_decode(qh, kpool, vpool, tab, np.array([p + 1], np.int32), Hkv, bs, scale)
        dt = (time.perf_counter() - t0) * layers
        line["cpu_baseline"] = {
            "value": round(nbytes / dt / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "tokens_per_s": round(P / dt, 2),
            "sample": ("oracle two-pass fp32 attention (restatement of src/layers/attention.cpp:"
                       "263-337) over one layer's 144 positions, scaled by 22 layers; the "
                       "append is not timed on the CPU")}
    print(json.dumps(line), flush=True)
    return 0


def run_prefill(steps: int, warmup: int):
    """cfg5's prefill compute: the 4 new sequences of a churn step, each with a
    2,048-token chunk at positions 0..2,047 (their whole context, in LIFO-reused
    blocks), causal prefill attention over the paged cache (skv_paged_prefill)
    at Llama-2-70B-style geometry.  The chunks are appended once before timing;
    a step is one skv_paged_prefill call over the 4 chunks.  Compute-bound:
    flops = 4 * sum over rows of (visible keys) * head_dim per query head
    (q.k and P.V, 2 flops per multiply-add), against MI355X's dense bf16 peak."""
    import stratakv_amd as skv

    skv.require_gpu()
    w = churn_workload(1)
    Hq, Hkv, hd, bs, total = w["Hq"], w["Hkv"], w["hd"], w["bs"], w["total"]
    nl, nn, chunk = CHURN_LONG, CHURN_NEW, CHURN_CHUNK
    tables = np.ascontiguousarray(w["tables"][nl:])
    mb = tables.shape[1]
    pool_elems = total * bs * Hkv * hd
    stream = skv.Stream()
    k_pool, v_pool = skv.DeviceBuffer(pool_elems * 2), skv.DeviceBuffer(pool_elems * 2)
    skv.fill_normal_bf16(k_pool, pool_elems, 0x5EED0505, 0, stream.handle)
    skv.fill_normal_bf16(v_pool, pool_elems, 0x5EED0506, 0, stream.handle)
    n_rows = nn * chunk
    ck, cv = skv.DeviceBuffer(n_rows * Hkv * hd * 2), skv.DeviceBuffer(n_rows * Hkv * hd * 2)
    skv.fill_normal_bf16(ck, n_rows * Hkv * hd, 0x5EED0507, 0, stream.handle)
    skv.fill_normal_bf16(cv, n_rows * Hkv * hd, 0x5EED0508, 0, stream.handle)
    q = skv.DeviceBuffer(n_rows * Hq * hd * 2)
    skv.fill_normal_bf16(q, n_rows * Hq * hd, 0x5EED0509, 0, stream.handle)
    dt = skv.DeviceBuffer.from_numpy(tables)
    zero = skv.DeviceBuffer.from_numpy(np.zeros(nn, np.int32))
    skv.kv_append(ck, cv, skv.DTYPE_BF16, k_pool, v_pool, total, dt, mb, zero, nn, chunk, Hkv, hd, bs,
                  stream=stream.handle)
    offsets = skv.DeviceBuffer.from_numpy((np.arange(nn + 1) * chunk).astype(np.int32))
    lens = skv.DeviceBuffer.from_numpy(np.full(nn, chunk, np.int32))
    out = skv.DeviceBuffer(n_rows * Hq * hd * 4)
    scale = 1.0 / math.sqrt(hd)

    def call():
        skv.paged_prefill(q, skv.DTYPE_BF16, k_pool, v_pool, total, dt, mb, offsets, lens, nn, n_rows,
                          Hq, Hkv, hd, bs, scale, out, stream=stream.handle)

    for _ in range(warmup):
        call()
    skv.synchronize()
    e0, e1 = skv.Event(), skv.Event()
    e0.record(stream.handle)
    for _ in range(steps):
        call()
    e1.record(stream.handle)
    skv.synchronize()
    ms = e0.elapsed_ms(e1) / steps
    visible = nn * chunk * (chunk + 1) // 2            # keys seen by the rows, summed
    flops = 4 * visible * Hq * hd
    tflops = flops / (ms / 1e3) / 1e12
    kv_bytes = nn * chunk * 2 * Hkv * hd * 2
    print(json.dumps({
        "metric": "paged prefill attention TFLOP/s (cfg5 prefill chunks)", "value": round(tflops, 2),
        "unit": "TFLOP/s", "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (device counter-hash N(0,1) bf16 Q/K/V, seeded)",
        "config": {"workload": ("cfg5 prefill: 4 sequences x 2,048-token chunks at positions "
                                "0..2,047 (LIFO-reused blocks), 64 Q / 8 KV heads, head_dim 128, "
                                "causal"), "chunk_tokens": chunk, "sequences": nn},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": 2500.0,
                     "unit": "TFLOP/s", "frac": round(tflops / 2500.0, 4),
                     "traffic": profile_traffic("cfg5", "prefill"),
                     "algorithmic_flops": flops,
                     "note": ("Q.K^T in bf16 and P.V in fp16 (V converted exactly as it is "
                              "staged, P rounded to fp16) on the matrix cores with fp32 "
                              "accumulation: they execute the algorithmic flops")},
        "kv_gbs": round(kv_bytes / (ms / 1e3) / 1e9, 2),
    }), flush=True)
    return 0


def cpu_compare(reps: int = 5):
    """The CPU baseline's two candidates, 1 thread each, at cfg2 geometry (one
    sequence, 32 Q / 4 KV heads, head_dim 64, context 4,097): the oracle's
    decode loops (the restatement of src/layers/attention.cpp:263-337, on an
    fp32 pool like the reference's cache and on a bf16 pool like this
    build's) against the reference's own single-token PagedAttention::forward
    (oracle/_ref), whose attention time is its time at context 4,097 minus its
    time at context 1 (the four identity projections, RoPE and the cache write
    are the same in both)."""
    import oracle

    Hq, Hkv, hd, bs, L = 32, 4, 64, 16, 4097
    rng = np.random.default_rng(0x5EED0002)
    nb = -(-L // bs)
    tables = rng.permutation(nb + 8)[:nb].astype(np.int32).reshape(1, nb)
    k32 = rng.standard_normal((nb + 8, bs, Hkv, hd), dtype=np.float32)
    v32 = rng.standard_normal((nb + 8, bs, Hkv, hd), dtype=np.float32)
    k16, v16 = oracle.f32_to_bf16(k32), oracle.f32_to_bf16(v32)
    q = rng.standard_normal((1, Hq, hd), dtype=np.float32)
    lens = np.array([L], np.int32)

    def median_ms(fn):
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append((time.perf_counter() - t0) * 1e3)
        return float(np.median(ts))

    scale = 1.0 / math.sqrt(hd)
    o32 = median_ms(lambda: oracle.paged_decode(q, k32, v32, tables, lens, Hkv, bs, scale))
    o16 = median_ms(lambda: oracle.paged_decode(q, k16, v16, tables, lens, Hkv, bs, scale, threads=1))
    line = {"cpu_compare": "cfg2 geometry: 1 sequence, 32 Q / 4 KV heads, head_dim 64, context 4,097, "
                           "1 thread, median of %d" % reps,
            "oracle_fp32_pool_ms": round(o32, 4), "oracle_bf16_pool_ms": round(o16, 4)}
    try:
        full, one = oracle.ref_decode_timing(Hq * hd, Hq, Hkv, bs, L, reps)
        line.update(reference_forward_ctx4097_ms=round(full, 4), reference_forward_ctx1_ms=round(one, 4),
                    reference_attention_ms=round(full - one, 4),
                    reference_over_oracle_fp32=round((full - one) / o32, 3))
    except (OSError, RuntimeError) as e:
        line["reference"] = f"unavailable: {e}"
    print(json.dumps(line), flush=True)
    return 0


# The kernel sources behind each traffic summary: the file with the kernels and
# the device headers it includes (the C ABI header declares no device code).
TRAFFIC_SOURCES = {"decode": ("skv_decode.hip", "skv_append.h", "skv_common.h"),
                   "prefill": ("skv_prefill.hip", "skv_common.h")}


def kernel_fingerprint(kind: str) -> str:
    """First 16 hex digits of the SHA-256 of the kernel sources of `kind`, in
    TRAFFIC_SOURCES order: what a counter summary was measured on."""
    h = hashlib.sha256()
    for name in TRAFFIC_SOURCES[kind]:
        with open(os.path.join(ROOT, "stratakv_amd", "csrc", name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def profile_traffic(workload_key: str, kind: str = "decode"):
    """HBM bytes per launch of the measured kernel(s) from the committed
    rocprof counter summary profiles/<kind>_traffic_<workload_key>.md, if one
    exists for this workload and was measured on the current kernel sources
    (its kernel_sources_sha256 line equals kernel_fingerprint(kind)); None
    otherwise, with the reason on stderr."""
    path = os.path.join(ROOT, "profiles", f"{kind}_traffic_{workload_key}.md")
    if not os.path.exists(path):
        return None
    text = open(path).read()
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", text)
    f = re.search(r"kernel_sources_sha256:\s*([0-9a-f]+)", text)
    current = kernel_fingerprint(kind)
    if not m or not f or f.group(1) != current:
        log(f"{os.path.basename(path)} was measured on other kernel sources "
            f"({f.group(1) if f else 'no fingerprint'}, now {current}): traffic reported as null")
        return None
    return float(m.group(1))


def copy_calibration(mib: int) -> int:
    """Copy `mib` MiB with the block-gather kernel (identity table, 1 MiB
    blocks): a plain copy of known size (reads and writes `mib` MiB once per
    launch), to scale the FETCH_SIZE / WRITE_SIZE counters."""
    import stratakv_amd as skv

    skv.require_gpu()
    block = 1 << 19  # bf16 elements = 1 MiB
    src = skv.DeviceBuffer(mib << 20)
    dst = skv.DeviceBuffer(mib << 20)
    skv.fill_normal_bf16(src, mib * block, 1)
    table = skv.DeviceBuffer.from_numpy(np.arange(mib, dtype=np.int32))
    for _ in range(5):
        skv.gather_blocks(src, mib, table, mib, block, dst)
    skv.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": mib << 20, "bytes_written": mib << 20,
                      "launches": 5}), flush=True)
    return 0


def read_calibration(gib: int, steps: int, warmup: int) -> int:
    """Plain streaming reads (skv_stream_read_checksum: one contiguous buffer,
    the decode's non-temporal 16-byte loads, 4 MiB chunks per wavefront) of
    `gib` GiB, timed with events on the launch stream: the rate reads alone
    reach on this GPU, the ceiling beside the decode's own load pattern."""
    import stratakv_amd as skv

    skv.require_gpu()
    nbytes = gib << 30
    data = skv.DeviceBuffer(nbytes)
    skv.fill_normal_bf16(data, nbytes // 2, 3)
    out = skv.DeviceBuffer(4)
    stream = skv.Stream()
    h = stream.handle
    for _ in range(warmup):
        skv.stream_read_checksum(data, nbytes, out, stream=h)
    ev = [skv.Event() for _ in range(steps + 1)]
    ev[0].record(h)
    for i in range(steps):
        skv.stream_read_checksum(data, nbytes, out, stream=h)
        ev[i + 1].record(h)
    skv.synchronize()
    ms = np.array([ev[i].elapsed_ms(ev[i + 1]) for i in range(steps)])
    print(json.dumps({"read_calibration_bytes": nbytes, "launches": steps,
                      "read_us": round(float(ms.mean()) * 1e3, 1),
                      "read_gbs": round(nbytes / (float(ms.mean()) / 1e3) / 1e9, 1),
                      "read_gbs_best": round(nbytes / (float(ms.min()) / 1e3) / 1e9, 1),
                      "frac_of_8tbs": round(nbytes / (float(ms.mean()) / 1e3) / 8e12, 4)}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=4, help="BASELINE.json config (1, 2, 3, 4 or 5)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--prefill", action="store_true",
                    help="with --config 5: time the chunked prefill attention of its 4 new "
                         "sequences (skv_paged_prefill) instead of the decode step")
    ap.add_argument("--separate", action="store_true",
                    help="time the decode-token append and the decode as two calls "
                         "(skv_kv_append + skv_paged_decode) instead of the fused call")
    ap.add_argument("--copy-calibration", type=int, metavar="MIB", default=0,
                    help="only run a plain copy of MIB MiB (counter calibration) and exit")
    ap.add_argument("--read-calibration", type=int, metavar="GIB", default=0,
                    help="only time plain streaming reads of GIB GiB (skv_stream_read_checksum) and exit")
    ap.add_argument("--load-calibration", action="store_true",
                    help="time the decode's load pattern alone (skv_paged_block_checksum) beside the "
                         "decode call on the --config 2-5 inputs, and exit")
    ap.add_argument("--contiguous-tables", action="store_true",
                    help="with --load-calibration --config 2, 3 or 4: the same lengths with each "
                         "sequence's blocks consecutive in a pool of the blocks used")
    ap.add_argument("--kernel-fingerprint", choices=sorted(TRAFFIC_SOURCES),
                    help="print the fingerprint of the decode or prefill kernel sources that a "
                         "traffic summary under profiles/ records, and exit")
    ap.add_argument("--cpu-compare", action="store_true",
                    help="time the oracle's decode loops against the reference's own attention "
                         "(oracle/_ref), 1 thread, at cfg2 geometry, and exit (CPU only)")
    args = ap.parse_args()
    if args.kernel_fingerprint:
        print(kernel_fingerprint(args.kernel_fingerprint))
        return 0
    if args.cpu_compare:
        return cpu_compare()
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    if args.read_calibration:
        return read_calibration(args.read_calibration, args.steps, args.warmup)
    if args.load_calibration:
        if args.config not in (2, 3, 4, 5):
            raise SystemExit("bench.py: --load-calibration runs on --config 2, 3, 4 or 5")
        w = workload(args.config)
        if args.contiguous_tables:
            if args.config == 5:
                raise SystemExit("bench.py: --contiguous-tables applies to --config 2, 3 or 4")
            w = contiguous_tables(w)
        log(w["desc"])
        return run_load_calibration(w, args.steps, args.warmup)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}). The paged "
              f"decode path shards by sequence or KV head with no exchange inside attention; that "
              f"design is not built or measured here.", file=sys.stderr)
        return 2
    if args.prefill:
        if args.config != 5:
            raise SystemExit("bench.py: --prefill measures config 5's prefill chunks (--config 5)")
        return run_prefill(args.steps, args.warmup)
    if args.config == 1:
        return run_cfg1(args.steps, args.warmup, not args.no_cpu_baseline)
    w = churn_workload(args.warmup + 2 * args.steps) if args.config == 5 else workload(args.config)
    dec_bytes, tok_bytes, churn_bytes, flops = algorithmic_bytes(w)
    log(w["desc"])
    log(f"algorithmic bytes per step: decode {dec_bytes / 1e9:.3f} GB + decode-token append "
        f"{tok_bytes / 1e6:.3f} MB + churn {churn_bytes / 1e6:.3f} MB")
    fused = not args.separate
    g = run_gpu(w, args.steps, args.warmup, fused=fused)
    step_s = g["ms_per_step"] / 1e3
    value = (dec_bytes + tok_bytes + churn_bytes) / step_s / 1e9
    main_bytes = dec_bytes + (tok_bytes if fused else 0)
    # The roofline's time: the timed region's own time per step when the step
    # is the decode call alone (fused append + decode, configs 2-4); with work
    # before the call (cfg5's churn, or --separate) the call's mean time from
    # the second, per-step-event pass.
    call_only = fused and "churn" not in w
    roof_s = step_s if call_only else g["main_ms"] / 1e3
    achieved = main_bytes / roof_s / 1e9
    per_call = main_bytes / (g["main_ms"] / 1e3) / 1e9
    key = f"cfg{args.config}" + ("" if fused else "_separate")
    traffic = profile_traffic(key)
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (device counter-hash N(0,1) bf16 K/V/Q, seeded)",
        "config": {
            "workload": w["desc"],
            "batch": w["B"], "num_q_heads": w["Hq"], "num_kv_heads": w["Hkv"],
            "head_dim": w["hd"], "block_size": w["bs"],
            "context_tokens_total": int(w["lens"].sum()),
            "context_min": int(w["lens"].min()), "context_max": int(w["lens"].max()),
            "accumulate": "fp32", "parallelism": "none (1 GPU)",
        },
        "tokens_per_s": round(w["B"] / step_s, 1),
        "hbm_frac_of_peak": round(value / HBM_PEAK_GBS, 4),
        "step": ("fused: skv_paged_decode_append (decode-token append + attention + merge)"
                 if fused else "separate: skv_kv_append, then skv_paged_decode")
                + ("; before it the churn table patch and 4 x 2,048-token chunk append"
                   if "churn" in w else ""),
        "pre_ms": round(g["pre_ms"], 5),
        "decode_ms": round(g["main_ms"], 5),
        "roofline": {
            "bound": "hbm",
            "kernel": ("skv_paged_decode_append: fused append + attention kernel, then merge"
                       if fused else "skv_paged_decode: attention kernel, then merge"),
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "algorithmic_bytes": main_bytes,
            "flops": flops,
            "time_source": ("timed region, ms_per_step" if call_only else
                            "mean decode-call time of a second pass with events around each call"),
            "achieved_per_call_events": round(per_call, 2),
        },
    }
    if not args.no_cpu_baseline:
        one, allc = cpu_baseline(w)
        line["cpu_baseline"] = one
        line["cpu_baseline_all_cores"] = allc
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
