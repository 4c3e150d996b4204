"""Score + compact throughput of the ActKV eviction step on one MI355X.

    python bench.py [--steps K] [--warmup W] [--layers 36] [--seq 32768] [--queries 128]

Workload (defaults): a Qwen3-8B-shaped paged cache -- 36 layers, 32 query / 8 KV heads,
head_dim 128, block_size 16, bf16 K/V ~ N(0,1) from a seed, physical blocks randomly permuted
-- holding one 32768-token sequence.  One step is the whole eviction pass:

  cal_attn : 128 action queries (bf16) with exact per-query lse, every layer, one launch
  evict    : keep mask = 4 sinks + top 10% by the layer-averaged head-mean score, then the
             conflict-free in-place compaction of all 72 K/V planes and block reclaim

Inputs are resident in HBM when a step starts.  Compaction mutates the cache, so every step
starts from a restored copy (device copy of kv + the host lists), outside the timed region;
the restore also overwrites the 256 MB MALL.  Each step is timed with HIP events on the
current stream (the library's launch stream), its launches queued behind the restore copy so
the interval is the GPU's time for the step; the scoring interval inside it is the duration of
the scoring call the roofline uses.  The same steps timed with the host's launch work exposed
(a synchronisation before each step) are reported beside it.

The single JSON line also carries the same numbers for one layer (the 32k-token one-layer
workload), the CPU baseline (the oracle's reference-style torch path on this host: the one
32k-token layer in full, median of --cpu-runs runs, scaled linearly to 36 layers for the whole
step), checks of the step's results and, under `configs`, the other workloads of the metric:
  cfg1 : one fp16 layer of 2048 tokens, 64 action queries, keep 25% + 4 sinks (with its CPU
         baseline in full)
  cfg3 : 36 layers x 8 ragged sequences of 8k-64k tokens, 64-256 action queries, keep 5-30%
         + 4 sinks, one shared shuffled pool; one cal_attn + one evict_batch (CPU baseline:
         one layer of one request, extrapolated and labelled so)
  cfg4 : 131072 tokens x 36 layers, keep mask of clustered runs, compaction only (CPU
         baseline: one layer's planes, extrapolated and labelled so)
each with its step time, algorithmic bytes and flops, GB/s, its floor and checks against the
oracle.  The agent loop (`ora`) runs all 50 rounds of its schedule.
"""
from __future__ import annotations

import argparse
import gc
import json
import math
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "actkv-open_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def parse(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--seq", type=int, default=32768)
    ap.add_argument("--queries", type=int, default=128)
    ap.add_argument("--q-heads", type=int, default=32)
    ap.add_argument("--kv-heads", type=int, default=8)
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--block-size", type=int, default=16)
    ap.add_argument("--keep", type=float, default=0.10)
    ap.add_argument("--sinks", type=int, default=4)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-runs", type=int, default=3, help="runs of each CPU baseline (median reported)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-single-layer", action="store_true", help="skip the one-layer measurement")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "score_kernel_traffic.json"),
                    help="rocprofv3 FETCH_SIZE/WRITE_SIZE summary of the scoring kernel (JSON)")
    ap.add_argument("--out", help="also write the JSON line here")
    ap.add_argument("--ora", action="store_true",
                    help="run the agent-loop workload instead (rounds of append + causal action scoring + "
                         "LRFU keep + compaction on a 36-layer batch of 4) and print its own JSON line")
    ap.add_argument("--ora-rounds", type=int, default=50)
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the 2k fp16, 36-layer ragged batch and 131k compaction legs")
    ap.add_argument("--configs-only", action="store_true",
                    help="run only those legs (cfg1 without its CPU baseline, cfg3, cfg4); one JSON line")
    ap.add_argument("--ora-short", type=int, default=50,
                    help="rounds of the agent-loop workload reported in the default JSON line (0: none)")
    ap.add_argument("--no-table1", action="store_true", help="skip the reference bench's Table-1 cases")
    ap.add_argument("--no-power", action="store_true", help="skip the power and clock reading")
    ap.add_argument("--no-gc-freeze", action="store_true",
                    help="agent loop: leave the startup heap in the collected generations (by default it "
                         "is frozen after setup, as a serving process does after loading)")
    ap.add_argument("--attn", action="store_true",
                    help="measure the paged attention kernel (the lse producer) instead: the 36-layer "
                         "32k-token cache with 128 queries, plain and causal, and a batch-8 decode step")
    ap.add_argument("--serve", action="store_true",
                    help="serve a Qwen3-8B-shaped model (random bf16 weights) on the paged cache through "
                         "the transformers backend: batch prefill, decode rounds with action tokens, ActKV "
                         "compression at each round's end; prints its own JSON line")
    ap.add_argument("--serve-batch", type=int, default=4)
    ap.add_argument("--serve-prompt", type=int, default=8192)
    ap.add_argument("--serve-rounds", type=int, default=4)
    ap.add_argument("--serve-steps", type=int, default=48, help="decode steps per round")
    ap.add_argument("--serve-action", type=int, default=24, help="action tokens at the end of each round")
    ap.add_argument("--serve-budget", type=int, default=4096)
    ap.add_argument("--serve-eager", action="store_true",
                    help="serve: launch every decode step from Python instead of replaying a HIP graph")
    args = ap.parse_args(argv)
    if args.steps < 1:
        ap.error("--steps must be at least 1 (the timed steps)")
    if args.warmup < 0:
        ap.error("--warmup must not be negative")
    if args.ora_short < 0:
        ap.error("--ora-short must not be negative")
    if args.ora_rounds < 1 or args.serve_rounds < 1 or args.serve_steps < 1:
        ap.error("--ora-rounds, --serve-rounds and --serve-steps must be at least 1")
    if not 0 <= args.serve_action <= args.serve_steps:
        ap.error("--serve-action must be between 0 and --serve-steps")
    return args


def run_info(torch, dev):
    """What ran: the GPU, the library build the kernels came from, and peak device memory."""
    from actkv import _hip
    return {"gpu": torch.cuda.get_device_name(dev),
            "kernels": f"{_hip.lib().actkv_version().decode()} ({os.path.basename(_hip.LIB_PATH)})",
            "peak_device_memory_bytes": int(torch.cuda.max_memory_allocated(dev))}


class Workload:
    """Seeded synthetic cache + action queries with exact lse, and a restorable snapshot.
    One sequence of `seq` tokens (default --seq) in `layers` layers; `queries` action queries
    (default --queries), keep ratio `keep` (default --keep) + --sinks, cache dtype `dtype`
    (default bf16); the physical blocks are drawn from a shuffled pool."""

    def __init__(self, args, layers, device, *, seq=None, queries=None, keep=None, dtype=None):
        import torch
        from actkv.paged import PagedKVCache

        self.args, self.L, self.dev = args, layers, device
        S = args.seq if seq is None else seq
        bs, hkv, hq, d = args.block_size, args.kv_heads, args.q_heads, args.head_dim
        self.dtype = torch.bfloat16 if dtype is None else dtype
        self.S, self.bs, self.hkv, self.hq, self.d = S, bs, hkv, hq, d
        self.N = args.queries if queries is None else queries
        self.nb = math.ceil(S / bs) + 64
        gcpu = torch.Generator().manual_seed(args.seed)
        self.cache = PagedKVCache(self.nb, bs, hkv, d, n_layers=layers, dtype=self.dtype, device=device)
        self.cache.free = torch.randperm(self.nb, generator=gcpu).tolist()
        gdev = torch.Generator(device=device).manual_seed(args.seed + 1)
        k = torch.randn(layers, S, hkv, d, generator=gdev, device=device, dtype=self.dtype)
        v = torch.randn(layers, S, hkv, d, generator=gdev, device=device, dtype=self.dtype)
        self.cache.append(0, k, v)
        del k, v
        self.q = torch.randn(layers, 1, self.N, hq, d, generator=gdev, device=device, dtype=self.dtype)
        self.lse = self._exact_lse()
        self.kv0 = self.cache.kv.clone()
        self.host0 = (list(self.cache.free), {0: list(self.cache.tables[0])}, dict(self.cache.seq_used))
        self.table0_i32 = np.array(self.host0[1][0], dtype=np.int32)
        self.width = math.ceil(S / bs) * bs
        self.out = torch.zeros(layers, 1, hkv, self.width, device=device)
        self.n_seen = torch.zeros(1, dtype=torch.int32, device=device)
        self.budget = int((args.keep if keep is None else keep) * S)

    def _exact_lse(self):
        """lse[l, 0, n, h] = logsumexp_t scale * q . k_t over the whole prefix, float32 on the GPU."""
        import torch
        g = self.hq // self.hkv
        scale = self.d ** -0.5
        lse = torch.empty(self.L, 1, self.N, self.hq, device=self.dev)
        slots = self.cache.slot_map(0)
        for l in range(self.L):
            kflat = self.cache.kv[l, 0].reshape(-1, self.hkv, self.d)[slots].float()   # [S, Hkv, D]
            for h in range(self.hkv):
                kt = kflat[:, h].t().contiguous()                                      # [D, S]
                qh = self.q[l, 0, :, h * g:(h + 1) * g].float().reshape(-1, self.d)   # [N*G, D]
                lse[l, 0, :, h * g:(h + 1) * g] = torch.logsumexp((qh @ kt) * scale, -1).view(self.N, g)
        return lse

    def restore(self):
        """Back to the pre-eviction state: KV bytes, free list, block table (with the int32 mirror
        the cache keeps for its own tables), lengths, pins."""
        from actkv.paged import _Table
        self.cache.kv.copy_(self.kv0)
        free, tables, seq = self.host0
        self.cache.free = list(free)
        self.cache.tables = {0: _Table(tables[0], self.table0_i32.copy())}
        self.cache.seq_used = dict(seq)
        self.cache.pinned.clear()
        self.n_seen.zero_()

    def step(self, ev=None):
        """One eviction pass; ev = (start, scored, end) events recorded on the current stream
        (scored may be None: no marker between the scoring call and the eviction)."""
        if ev:
            ev[0].record()
        self.cache.cal_attn([0], self.q, self.lse, self.out, self.n_seen, layer=None)
        if ev and ev[1] is not None:
            ev[1].record()
        perm = self.cache.evict(0, self.out[:, 0], self.budget, protected=self.args.sinks)
        if ev:
            ev[2].record()
        return perm

    # ---------------------------------------------------------------- algorithmic work
    def algorithmic(self, moved_pairs, drop):
        L, S, hkv, hq, d, N, bs = self.L, self.S, self.hkv, self.hq, self.d, self.N, self.bs
        e = self.cache.kv.element_size()
        nblk = math.ceil(S / bs)
        per_layer_score = S * hkv * d * e + N * hq * d * e + N * hq * 4 + 2 * hkv * S * 4 + nblk * 4
        score = L * per_layer_score
        keep = L * hkv * S * 4 + S
        compact = moved_pairs * 2 * L * hkv * d * e * 2 + S + 2 * nblk * 4 + drop * 4
        flops = 2 * N * hq * S * d * L
        return {"bytes_score": score, "bytes_keep": keep, "bytes_compact": compact, "flops_score": flops,
                "bytes_score_per_layer": per_layer_score}


def measure(w, steps, warmup):
    """Time `steps` eviction steps between two device synchronisations.

    Each step starts from a restored cache.  The restore (a device copy of the whole cache) is
    queued first and the step's launches are queued behind it with no synchronisation, so the
    host prepares the step while the GPU copies, as a serving loop prepares step i+1 while step
    i runs.  Events on the launch stream at the step's start and end give the GPU's time for
    the step.  An event is a marker packet that itself holds the queue for several
    microseconds, so the split into the scoring call (kernel + n_seen bump) and the eviction
    comes from a second pass of the same steps with a third event between them (its two
    intervals add up to a little more than the step).

    The same steps are then timed once more with a synchronisation before each step, so the
    host's launch work is exposed; that figure is reported beside the first."""
    import torch
    E = lambda: torch.cuda.Event(enable_timing=True)
    for _ in range(warmup):
        w.restore()
        w.step()
    torch.cuda.synchronize()
    evs = []
    wall0 = time.perf_counter()
    for _ in range(steps):
        w.restore()
        ev = [E(), None, E()]
        w.step(ev)
        evs.append(ev)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    t_step = [e[0].elapsed_time(e[2]) * 1e3 for e in evs]
    evs = []
    for _ in range(steps):
        w.restore()
        ev = [E() for _ in range(3)]
        w.step(ev)
        evs.append(ev)
    torch.cuda.synchronize()
    t_score = [e[0].elapsed_time(e[1]) * 1e3 for e in evs]
    t_evict = [e[1].elapsed_time(e[2]) * 1e3 for e in evs]
    t_sync = []
    for _ in range(steps):
        w.restore()
        torch.cuda.synchronize()
        ev = [E(), None, E()]
        w.step(ev)
        torch.cuda.synchronize()
        t_sync.append(ev[0].elapsed_time(ev[2]) * 1e3)
    return {"step_us": statistics.mean(t_step), "step_us_median": statistics.median(t_step),
            "score_us": statistics.mean(t_score), "evict_us": statistics.mean(t_evict),
            "step_us_sync": statistics.mean(t_sync), "wall_s_incl_restore": wall}


def time_apply_copies(torch, w, moved, steps):
    """apply_copies (the explicit src/dst row mover, compaction.py:79-106) on the workload's
    cache with a plan of its compaction's size: `moved` rows of every plane (K and V of every
    layer) from distinct source slots to distinct destination slots, the two sets disjoint as
    plan_compaction makes them.  HIP events around back-to-back calls on the launch stream.
    Algorithmic bytes: every moved row read and written, plus the two int64 index arrays.
    Beside it, on the same GPU: the reference's torch formulations of the same move
    (apply_copies_ref, compaction.py:72-74) and of its gather baseline (gather_compaction,
    compaction.py:109-114: the survivors of a keep set of the compaction's size copied into a
    fresh buffer)."""
    from actkv.kernels.compaction import apply_copies, apply_copies_ref, gather_compaction
    kv = w.cache.kv
    planes = kv.shape[0] * kv.shape[1]
    flat = kv.view(planes, kv.shape[2] * kv.shape[3], kv.shape[4] * kv.shape[5])
    slots = flat.shape[1]
    g = torch.Generator().manual_seed(7)
    pick = torch.randperm(slots, generator=g)[: 2 * moved]
    src, dst = pick[:moved].to(w.dev), pick[moved:].to(w.dev)
    stream = torch.cuda.current_stream(w.dev)

    def timed(fn, reps):
        fn()
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        for _ in range(reps):
            fn()
        ev1.record(stream)
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) * 1e3 / reps

    us = timed(lambda: apply_copies(flat, src, dst), steps)
    us_ref = timed(lambda: apply_copies_ref(flat, src, dst), max(steps // 4, 3))
    keep = torch.sort(torch.randperm(slots, generator=g)[: w.budget + w.args.sinks]).values.to(w.dev)
    us_gather = timed(lambda: gather_compaction(flat, keep), max(steps // 4, 3))
    nbytes = 2 * moved * planes * flat.shape[2] * flat.element_size() + 2 * moved * 8
    gbytes = 2 * keep.numel() * planes * flat.shape[2] * flat.element_size() + keep.numel() * 8
    return {"workload": f"{moved} rows x {planes} planes of {flat.shape[2] * flat.element_size()} B, "
                        f"random disjoint source and destination slots", "us": round(us, 2),
            "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "frac_of_hbm_peak": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "bytes": nbytes,
            "kernel": "copy_slots_kernel (actkv_copy_slots)",
            "apply_copies_ref_torch_us": round(us_ref, 2),
            "gather_compaction_torch": {"kept_rows": keep.numel(), "us": round(us_gather, 2),
                                        "GBps": round(gbytes / (us_gather * 1e-6) / 1e9, 1)}}


def check_step(w):
    """Run one step from a fresh copy and check it: keep mask == the oracle's keep mask on the
    GPU's own scores; survivors of layer 0 == the pre-compaction rows at perm; host lists."""
    import numpy as np
    import torch
    from oracle import reference as ref

    w.restore()
    slots_before = w.cache.slot_map(0)
    perm = w.step()
    torch.cuda.synchronize()
    scores = w.out[:, 0].cpu()
    # the oracle's keep mask with the documented tie rule (lower index first), which equals
    # torch.topk's wherever the k-th and (k+1)-th candidate scores differ
    keep_o = ref.keep_mask_lowest_index_ties(scores, w.S, w.budget, protected=w.args.sinks)
    kept_o = torch.nonzero(keep_o).flatten()
    ok_mask = bool(torch.equal(torch.sort(perm.cpu()).values, kept_o))
    src, dst, perm_o, drop = ref.plan_compaction(keep_o.numpy(), w.S, w.host0[1][0], w.bs)
    ok_perm = bool(np.array_equal(perm.cpu().numpy(), perm_o))
    flat0 = w.kv0[0].view(2, -1, w.hkv, w.d)
    before = flat0[:, slots_before[perm]]
    after_slots = w.cache.slot_map(0)
    after = w.cache.kv[0].view(2, -1, w.hkv, w.d)[:, after_slots]
    ok_rows = bool(torch.equal(before.view(torch.int16), after.view(torch.int16)))
    nblk = math.ceil(w.S / w.bs)
    ok_host = (w.cache.seq_used[0] == int(keep_o.sum()) and len(w.cache.tables[0]) == nblk - drop
               and len(w.cache.free) == w.nb - (nblk - drop))
    ok_out = outputs_match(w, slots_before, keep_o)
    return {"keep_mask_matches_oracle": ok_mask, "perm_matches_oracle": ok_perm,
            "layer0_rows_match": ok_rows, "allocator_state_ok": ok_host,
            "outputs_match": ok_out}, int(src.size), int(drop)


def outputs_match(w, slots_before, keep):
    """The reference bench's attention check (benchmarks/bench_kernels.py:126-133): decode
    attention of a fresh query after the step equals the same attention over the gather
    baseline, within rtol = atol = 1e-3.  The compacted cache is attended by the paged
    attention kernel; the baseline is the pre-step cache's survivors (the oracle's keep mask on
    the step's scores) gathered into a fresh contiguous buffer (gather_compaction,
    compaction.py:109-114) and attended by the torch reference (lse_attn.py:42-60)."""
    import torch
    from actkv.kernels.compaction import gather_compaction
    from actkv.kernels.lse_attn import paged_decode_attention, paged_decode_attention_ref
    g = torch.Generator(device=w.dev).manual_seed(w.args.seed + 7)
    q2 = torch.randn(1, w.hq, w.d, generator=g, device=w.dev, dtype=w.dtype)
    seq, bt = w.cache._device_tables([0])
    got, _ = paged_decode_attention(q2, w.cache.kv[0], bt, seq)
    keep_slots = slots_before[torch.from_numpy(keep.numpy()).to(w.dev)]
    flat0 = w.kv0[0].view(2, -1, w.hkv * w.d)
    base = gather_compaction(flat0, keep_slots)                  # [2, B, Hkv*D]
    b = base.shape[1]
    nblk = -(-b // w.bs)
    pad = torch.zeros(2, nblk * w.bs - b, base.shape[2], dtype=base.dtype, device=w.dev)
    kv_base = torch.cat([base, pad], 1).view(2, nblk, w.bs, w.hkv, w.d)
    table = torch.arange(nblk, dtype=torch.int32, device=w.dev).view(1, -1)
    want, _ = paged_decode_attention_ref(q2, kv_base, table, torch.tensor([b], device=w.dev))
    return bool(torch.allclose(got, want, rtol=1e-3, atol=1e-3))


def extra_memory_mb(w):
    """Peak device memory one step allocates above what it started with (the reference bench's
    extra-memory column, benchmarks/bench_kernels.py:143-151), after a warm step."""
    import torch
    w.restore()
    w.step()
    w.restore()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(w.dev)
    base = torch.cuda.memory_allocated(w.dev)
    w.step()
    torch.cuda.synchronize()
    return round((torch.cuda.max_memory_allocated(w.dev) - base) / 2 ** 20, 3)


def power_leg(w, seconds=1.5):
    """Socket power and GFX clock while the scoring call runs back to back (amd-smi, sampled
    after a warm-up), and the dense bf16 matrix-core peak at that clock.  The scoring kernel
    runs at the board's power limit, so its clock, not the 2.4 GHz the 2.5 PFLOP/s peak is
    quoted at, bounds what the matrix cores can deliver.  None where amd-smi is missing."""
    import shutil
    import subprocess
    import torch
    smi = shutil.which("amd-smi")
    if not smi:
        return None
    w.restore()
    samples, calls = [], 0
    t0 = time.perf_counter()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            w.cache.cal_attn([0], w.q, w.lse, w.out, w.n_seen, layer=None)
        calls += 8
        el = time.perf_counter() - t0
        if el > 0.4 and len(samples) < 4 and el > 0.4 + 0.25 * len(samples):
            try:
                out = subprocess.run([smi, "metric", "-g", "0", "--json", "-p", "-c"], capture_output=True,
                                     text=True, timeout=10).stdout
                d = json.loads(out)
                g = d["gpu_data"][0] if isinstance(d, dict) else d[0]
                clks = [v["clk"]["value"] for k, v in g["clock"].items() if k.startswith("gfx_")]
                samples.append((float(g["power"]["socket_power"]["value"]), sum(clks) / len(clks)))
            except Exception:
                pass
    ev[1].record()
    torch.cuda.synchronize()
    call_us = ev[0].elapsed_time(ev[1]) * 1e3 / calls
    w.restore()
    if not samples:
        return None
    pw = sum(s[0] for s in samples) / len(samples)
    clk = sum(s[1] for s in samples) / len(samples)
    flops = w.algorithmic(0, 0)["flops_score"]
    peak_at_clk = BF16_PEAK_TFLOPS * clk / 2400.0
    achieved = flops / (call_us * 1e-6) / 1e12
    return {"source": "amd-smi metric, while the scoring call runs back to back", "samples": len(samples),
            "socket_power_w": round(pw, 1), "gfx_clock_mhz": round(clk, 1), "scoring_call_us": round(call_us, 2),
            "bf16_peak_at_clock_tflops": round(peak_at_clk, 1),
            "frac_of_peak_at_clock": round(achieved / peak_at_clk, 4)}


# The reference's published Table-1 step times (NVIDIA A100-SXM4-80GB, fp16, one layer, one
# action query; median of 5 after 1 warm-up): results/bench_kernels.txt:3-14 of the reference.
TABLE1_A100_MS = {(1024, 512, 1): 1.233, (1024, 512, 4): 4.128, (1024, 512, 16): 15.690, (1024, 512, 64): 61.856,
                  (2048, 1536, 1): 1.248, (2048, 1536, 4): 4.290, (2048, 1536, 16): 16.214, (2048, 1536, 64): 63.968,
                  (6144, 4096, 1): 1.394, (6144, 4096, 4): 4.753, (6144, 4096, 16): 18.111, (6144, 4096, 64): 71.083}


def run_table1(torch, dev, seed=0, warmup=1, iters=5):
    """The reference bench's Table-1 cases on this GPU, for context (benchmarks/bench_kernels.py:
    67-151): r requests of n tokens in one fp16 layer (32 q / 8 KV heads, head_dim 128, block 16,
    physical blocks shuffled), one action query per request with its lse from decode attention.
    A step is what the reference times: block table, cal_attn of the query, then evict of each
    request in a Python loop (paged.py:141-157); `batched_ms` is the same step with one
    evict_batch call.  Wall time with a synchronisation on both sides, median of `iters` steps on
    fresh caches after `warmup`, as the reference does."""
    from actkv.paged import PagedKVCache
    hq, hkv, d, bs = 32, 8, 128, 16

    def build(r, n):
        nb = r * math.ceil(n / bs) + 4
        cache = PagedKVCache(nb, bs, hkv, d, dtype=torch.float16, device=dev)
        cache.free = torch.randperm(nb, generator=torch.Generator().manual_seed(seed)).tolist()
        g = torch.Generator(device=dev).manual_seed(seed)
        k = torch.randn(1, r * n, hkv, d, generator=g, device=dev, dtype=torch.float16)
        v = torch.randn(k.shape, generator=g, device=dev, dtype=torch.float16)
        cache.append_batch(list(range(r)), k, v, [n] * r)
        return cache

    def step(cache, reqs, q, lse, budget, batched):
        bt = cache.block_table(reqs)
        out = torch.zeros(len(reqs), hkv, bt.shape[1] * bs, device=dev)
        nseen = torch.zeros(len(reqs), dtype=torch.int32, device=dev)
        cache.cal_attn(reqs, q, lse, out, nseen)
        if batched:
            cache.evict_batch(reqs, out, budget)
        else:
            for i in reqs:
                cache.evict(i, out[i], budget)

    def timed(r, n, reqs, q, lse, budget, batched):
        for _ in range(warmup):
            step(build(r, n), reqs, q, lse, budget, batched)
        times = []
        for _ in range(iters):
            cache = build(r, n)
            torch.cuda.synchronize()
            t = time.perf_counter()
            step(cache, reqs, q, lse, budget, batched)
            torch.cuda.synchronize()
            times.append((time.perf_counter() - t) * 1e3)
        return statistics.median(times)

    rows = []
    for (n, budget, r), a100 in TABLE1_A100_MS.items():
        reqs = list(range(r))
        q = torch.randn(r, hq, d, generator=torch.Generator(device=dev).manual_seed(1), device=dev,
                        dtype=torch.float16)
        probe = build(r, n)
        _, lse = probe.decode_attention(reqs, q)
        del probe
        ms = timed(r, n, reqs, q, lse, budget, False)
        ms_b = timed(r, n, reqs, q, lse, budget, True)
        rows.append({"n": n, "budget": budget, "r": r, "ms": round(ms, 3), "batched_ms": round(ms_b, 3),
                     "a100_published_ms": a100, "speedup_vs_a100": round(a100 / ms, 1)})
    return {"workload": "the reference bench's Table-1 cases: 1 fp16 layer, 32 q / 8 KV heads, head_dim 128, "
                        "block 16, one action query; step = cal_attn + evict per request (batched_ms: one "
                        "evict_batch); wall time, median of 5 after 1 warm-up",
            "cases": rows}


class RaggedWorkload:
    """A batch of ragged sequences in one shared, shuffled block pool: R requests of S_r ~
    U[8192, 65536] tokens in L layers, N_r ~ U[64, 256] action queries each (bf16, exact
    lse), keep ratio r_r ~ U[0.05, 0.30] + --sinks, all drawn from the seed.  One step scores
    every layer and request in one cal_attn (n_valid = N_r) and evicts every request in one
    evict_batch call."""

    def __init__(self, args, device, R=8, L=36):
        import torch
        from actkv.paged import PagedKVCache

        seed = args.seed + 3
        rng = np.random.default_rng(seed)
        bs, hkv, hq, d = args.block_size, args.kv_heads, args.q_heads, args.head_dim
        self.args, self.R, self.L, self.dev = args, R, L, device
        self.bs, self.hkv, self.hq, self.d, self.sinks = bs, hkv, hq, d, args.sinks
        self.S = [int(x) for x in rng.integers(8192, 65537, R)]
        self.Nq = [int(x) for x in rng.integers(64, 257, R)]
        self.ratio = [float(x) for x in rng.uniform(0.05, 0.30, R)]
        self.budgets = [int(r * s) for r, s in zip(self.ratio, self.S)]
        self.nb = sum(math.ceil(s / bs) for s in self.S) + 64
        self.cache = PagedKVCache(self.nb, bs, hkv, d, n_layers=L, dtype=torch.bfloat16, device=device)
        self.cache.free = torch.randperm(self.nb, generator=torch.Generator().manual_seed(seed)).tolist()
        gdev = torch.Generator(device=device).manual_seed(seed + 1)
        self.reqs = list(range(R))
        for r, n in enumerate(self.S):
            k = torch.randn(L, n, hkv, d, generator=gdev, device=device, dtype=torch.bfloat16)
            v = torch.randn(L, n, hkv, d, generator=gdev, device=device, dtype=torch.bfloat16)
            self.cache.append(r, k, v)
            del k, v
        nmax = max(self.Nq)
        self.q = torch.randn(L, R, nmax, hq, d, generator=gdev, device=device, dtype=torch.bfloat16)
        self.n_valid = torch.tensor(self.Nq, dtype=torch.int32, device=device)
        self.lse = self._exact_lse(nmax)
        self.kv0 = self.cache.kv.clone()
        self.host0 = (list(self.cache.free), {r: list(self.cache.tables[r]) for r in self.reqs},
                      dict(self.cache.seq_used))
        self.tables0_i32 = {r: np.array(self.host0[1][r], dtype=np.int32) for r in self.reqs}
        self.width = max(math.ceil(n / bs) for n in self.S) * bs
        self.out = torch.zeros(L, R, hkv, self.width, device=device)
        self.n_seen = torch.zeros(R, dtype=torch.int32, device=device)

    def _exact_lse(self, nmax):
        """lse[l, r, n, h] = logsumexp_t scale * q . k_t over request r's tokens (n < N_r),
        float32 on the GPU; rows n >= N_r are never read."""
        import torch
        g, scale = self.hq // self.hkv, self.d ** -0.5
        lse = torch.zeros(self.L, self.R, nmax, self.hq, device=self.dev)
        for r in self.reqs:
            slots, n = self.cache.slot_map(r), self.Nq[r]
            for l in range(self.L):
                kflat = self.cache.kv[l, 0].reshape(-1, self.hkv, self.d)[slots]
                for h in range(self.hkv):
                    kt = kflat[:, h].float().t().contiguous()
                    qh = self.q[l, r, :n, h * g:(h + 1) * g].float().reshape(-1, self.d)
                    lse[l, r, :n, h * g:(h + 1) * g] = torch.logsumexp((qh @ kt) * scale, -1).view(n, g)
        return lse

    def restore(self):
        from actkv.paged import _Table
        self.cache.kv.copy_(self.kv0)
        free, tables, seq = self.host0
        self.cache.free = list(free)
        self.cache.tables = {r: _Table(tables[r], self.tables0_i32[r].copy()) for r in self.reqs}
        self.cache.seq_used = dict(seq)
        self.cache.pinned.clear()
        self.n_seen.zero_()

    def step(self, ev=None):
        if ev:
            ev[0].record()
        self.cache.cal_attn(self.reqs, self.q, self.lse, self.out, self.n_seen, layer=None, n_valid=self.n_valid)
        if ev and ev[1] is not None:
            ev[1].record()
        perms = self.cache.evict_batch(self.reqs, self.out, self.budgets, protected=self.sinks)
        if ev:
            ev[2].record()
        return perms

    def algorithmic(self, moved, drops):
        L, hkv, hq, d, bs, e = self.L, self.hkv, self.hq, self.d, self.bs, 2
        score = keep = compact = flops = 0
        for S, N, m, dr in zip(self.S, self.Nq, moved, drops):
            nblk = math.ceil(S / bs)
            score += L * (S * hkv * d * e + N * hq * d * e + N * hq * 4 + 2 * hkv * S * 4 + nblk * 4)
            keep += L * hkv * S * 4 + S
            compact += m * 2 * L * hkv * d * e * 2 + S + 2 * nblk * 4 + dr * 4
            flops += 2 * N * hq * S * d * L
        return {"bytes_score": score, "bytes_keep": keep, "bytes_compact": compact, "flops_score": flops}


def check_ragged(w):
    """One step of the ragged batch against the oracle, request by request in order: keep mask
    (the oracle's on the GPU's own scores, equal scores at the boundary taken lower index
    first), perm (its compaction plan), the allocator (tables,
    the free list's order, lengths: paged.py:135-138 applied sequentially) and the survivors'
    K/V rows of the first and last layer at perm."""
    import torch
    from oracle import reference as ref

    w.restore()
    slots_before = {r: w.cache.slot_map(r) for r in w.reqs}
    perms = w.step()
    torch.cuda.synchronize()
    scores = w.out.cpu()
    free, tables, seq = list(w.host0[0]), {r: list(t) for r, t in w.host0[1].items()}, {}
    ok_mask = ok_perm = ok_rows = True
    moved, drops = [], []
    for i, r in enumerate(w.reqs):
        S = w.S[i]
        keep_o = ref.keep_mask_lowest_index_ties(scores[:, i, :, :S], S, w.budgets[i], protected=w.sinks)
        src, _, perm_o, drop = ref.plan_compaction(keep_o.numpy(), S, tables[r], w.bs)
        moved.append(int(src.size))
        drops.append(int(drop))
        p = perms[i].cpu()
        ok_mask = ok_mask and bool(torch.equal(torch.sort(p).values, torch.nonzero(keep_o).flatten()))
        ok_perm = ok_perm and bool(np.array_equal(p.numpy(), perm_o))
        free.extend(reversed(tables[r][:drop]))
        tables[r] = tables[r][drop:]
        seq[r] = int(keep_o.sum())
        pd = perms[i]
        after_slots = w.cache.slot_map(r)
        for l in (0, w.L - 1):
            before = w.kv0[l].view(2, -1, w.hkv, w.d)[:, slots_before[r][pd]]
            after = w.cache.kv[l].view(2, -1, w.hkv, w.d)[:, after_slots]
            ok_rows = ok_rows and bool(torch.equal(before.view(torch.int16), after.view(torch.int16)))
    ok_host = (w.cache.free == free and {r: list(w.cache.tables[r]) for r in w.reqs} == tables
               and w.cache.seq_used == seq)
    return {"keep_masks_match_oracle": ok_mask, "perms_match_oracle": ok_perm,
            "first_last_layer_rows_match": ok_rows, "allocator_state_matches_oracle": ok_host}, moved, drops


class ClusteredWorkload:
    """One sequence of S tokens in L layers (bf16, shuffled pool) and a keep mask drawn as
    alternating runs: kept runs Geom(mean 32), dropped runs Geom(mean 128), overall keep about
    0.2.  One step is PagedKVCache.compact with that mask (paged.py:125-139): plan, row moves of
    every layer's K and V, block reclaim."""

    def __init__(self, args, device, S=131072, L=36):
        import torch
        from actkv.paged import PagedKVCache

        seed = args.seed + 5
        bs, hkv, d = args.block_size, args.kv_heads, args.head_dim
        self.args, self.S, self.L, self.dev, self.bs, self.hkv, self.d = args, S, L, device, bs, hkv, d
        self.nb = math.ceil(S / bs) + 64
        self.cache = PagedKVCache(self.nb, bs, hkv, d, n_layers=L, dtype=torch.bfloat16, device=device)
        self.cache.free = torch.randperm(self.nb, generator=torch.Generator().manual_seed(seed)).tolist()
        gdev = torch.Generator(device=device).manual_seed(seed + 1)
        k = torch.randn(L, S, hkv, d, generator=gdev, device=device, dtype=torch.bfloat16)
        v = torch.randn(L, S, hkv, d, generator=gdev, device=device, dtype=torch.bfloat16)
        self.cache.append(0, k, v)
        del k, v
        rng = np.random.default_rng(seed)
        mask = np.zeros(S, dtype=bool)
        t, kept_run = 0, True
        while t < S:
            n = int(rng.geometric(1 / 32 if kept_run else 1 / 128))
            if kept_run:
                mask[t:t + n] = True
            t += n
            kept_run = not kept_run
        self.keep_host = torch.from_numpy(mask)
        self.keep = self.keep_host.to(device)
        self.kv0 = self.cache.kv.clone()
        self.host0 = (list(self.cache.free), {0: list(self.cache.tables[0])}, dict(self.cache.seq_used))
        self.table0_i32 = np.array(self.host0[1][0], dtype=np.int32)

    def restore(self):
        from actkv.paged import _Table
        self.cache.kv.copy_(self.kv0)
        free, tables, seq = self.host0
        self.cache.free = list(free)
        self.cache.tables = {0: _Table(tables[0], self.table0_i32.copy())}
        self.cache.seq_used = dict(seq)
        self.cache.pinned.clear()

    def step(self, ev=None):
        if ev:
            ev[0].record()
        perm = self.cache.compact(0, self.keep)
        if ev:
            ev[2].record()
        return perm

    def algorithmic(self, moved, drop):
        nblk = math.ceil(self.S / self.bs)
        return {"bytes_compact": moved * 2 * self.L * self.hkv * self.d * 2 * 2 + self.S + 2 * nblk * 4 + drop * 4}


def check_clustered(w):
    """The compaction against the oracle: perm (its plan), the allocator, and the first and last
    layers' survivors at perm."""
    import torch
    from oracle import reference as ref

    w.restore()
    slots_before = w.cache.slot_map(0)
    perm = w.step()
    torch.cuda.synchronize()
    src, _, perm_o, drop = ref.plan_compaction(w.keep_host.numpy(), w.S, w.host0[1][0], w.bs)
    ok_perm = bool(np.array_equal(perm.cpu().numpy(), perm_o))
    table = w.host0[1][0]
    free = list(w.host0[0]) + list(reversed(table[:drop]))
    ok_host = (w.cache.free == free and list(w.cache.tables[0]) == table[drop:]
               and w.cache.seq_used[0] == int(w.keep_host.sum()))
    after_slots = w.cache.slot_map(0)
    ok_rows = True
    for l in (0, w.L - 1):
        before = w.kv0[l].view(2, -1, w.hkv, w.d)[:, slots_before[perm]]
        after = w.cache.kv[l].view(2, -1, w.hkv, w.d)[:, after_slots]
        ok_rows = ok_rows and bool(torch.equal(before.view(torch.int16), after.view(torch.int16)))
    return {"perm_matches_oracle": ok_perm, "allocator_state_matches_oracle": ok_host,
            "first_last_layer_rows_match": ok_rows}, int(src.size), int(drop)


def time_steps(w, steps, warmup):
    """Events at each step's start and end, every step from a restored copy (as measure())."""
    import torch
    for _ in range(warmup):
        w.restore()
        w.step()
    torch.cuda.synchronize()
    evs = []
    for _ in range(steps):
        w.restore()
        ev = [torch.cuda.Event(enable_timing=True), None, torch.cuda.Event(enable_timing=True)]
        w.step(ev)
        evs.append(ev)
    torch.cuda.synchronize()
    t = [e[0].elapsed_time(e[2]) * 1e3 for e in evs]
    return {"step_us": statistics.mean(t), "step_us_median": statistics.median(t)}


def roof(bytes_hbm, flops=0):
    """Floor of a phase: its HBM bytes at 8 TB/s or its dense bf16 flops at 2.5 PFLOP/s."""
    return max(bytes_hbm / (HBM_PEAK_GBS * 1e9), flops / (BF16_PEAK_TFLOPS * 1e12)) * 1e6


def run_cfg1(args, dev, cpu=True):
    """The reference's CPU-runnable case on the GPU: one fp16 layer, one 2048-token sequence,
    64 action queries with exact lse, keep 25% (budget 512) + 4 sinks, shuffled blocks; scoring
    then evict.  Checks as the headline step's; the CPU baseline times the same case in full."""
    import torch
    w = Workload(args, 1, dev, seq=2048, queries=64, keep=0.25, dtype=torch.float16)
    checks, moved, drop = check_step(w)
    work = w.algorithmic(moved, drop)
    m = measure(w, max(args.steps, 10), max(args.warmup, 2))
    nbytes = work["bytes_score"] + work["bytes_keep"] + work["bytes_compact"]
    floor = roof(work["bytes_score"], work["flops_score"]) + roof(work["bytes_keep"] + work["bytes_compact"])
    res = {"workload": "1 layer x 1 sequence x 2048 tokens, Hq 32 / Hkv 8, head_dim 128, block 16, fp16, "
                       "64 action queries, keep 25% (budget 512) + 4 sinks, shuffled blocks",
           "step_us": round(m["step_us"], 2), "step_us_median": round(m["step_us_median"], 2),
           "score_us": round(m["score_us"], 2), "evict_us": round(m["evict_us"], 2),
           "algorithmic": work, "GBps": round(nbytes / (m["step_us"] * 1e-6) / 1e9, 1),
           "pct_of_hbm_peak": round(100 * nbytes / (m["step_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 3),
           "bound": "hbm", "floor_us": round(floor, 2), "frac_of_floor": round(floor / m["step_us"], 4),
           "checks": checks}
    if cpu:
        res["cpu_baseline"] = cpu_summary(cpu_runs(w, 3), nbytes, "the whole case (one fp16 layer, 2048 tokens, 64 action queries)")
    del w
    return res


def run_cfg3(args, dev, steps=5, cpu=False):
    """36 layers x 8 ragged sequences scored and evicted in one cal_attn + one evict_batch.
    cpu: also time the CPU baseline on one layer of one request, extrapolated (labelled)."""
    w = RaggedWorkload(args, dev)
    checks, moved, drops = check_ragged(w)
    work = w.algorithmic(moved, drops)
    m = measure(w, steps, 1)
    nbytes = work["bytes_score"] + work["bytes_keep"] + work["bytes_compact"]
    floor_score = roof(work["bytes_score"], work["flops_score"])
    floor = floor_score + roof(work["bytes_keep"] + work["bytes_compact"])
    res = {"workload": f"{w.L} layers x {w.R} ragged sequences of {min(w.S)}-{max(w.S)} tokens "
                       f"(sum {sum(w.S)}), Hq 32 / Hkv 8, head_dim 128, block 16, bf16, "
                       f"{min(w.Nq)}-{max(w.Nq)} action queries, keep {min(w.ratio):.1%}-{max(w.ratio):.1%} "
                       f"+ {w.sinks} sinks, one shared shuffled block pool; one cal_attn + one evict_batch",
           "seq_lens": w.S, "action_queries": w.Nq, "budgets": w.budgets,
           "step_us": round(m["step_us"], 1), "step_us_median": round(m["step_us_median"], 1),
           "score_us": round(m["score_us"], 1), "evict_us": round(m["evict_us"], 1),
           "evict_us_per_layer": round(m["step_us"] / w.L, 2),
           "algorithmic": work, "GBps": round(nbytes / (m["step_us"] * 1e-6) / 1e9, 1),
           "pct_of_hbm_peak": round(100 * nbytes / (m["step_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 2),
           "score_TFLOPs": round(work["flops_score"] / (m["score_us"] * 1e-6) / 1e12, 1),
           "bound": ("mfma" if work["flops_score"] / (BF16_PEAK_TFLOPS * 1e12)
                     > work["bytes_score"] / (HBM_PEAK_GBS * 1e9) else "hbm"),
           "floor_us": round(floor, 1), "frac_of_floor": round(floor / m["step_us"], 4),
           "moved_rows": sum(moved), "blocks_freed": sum(drops), "checks": checks}
    if cpu:
        res["cpu_baseline"] = cpu_ragged(w, nbytes)
    del w
    return res


def run_cfg4(args, dev, steps=5, cpu=False):
    """131072 tokens x 36 layers, clustered keep runs, compaction only.  cpu: also time the
    CPU baseline on one layer's planes, extrapolated to every layer (labelled)."""
    w = ClusteredWorkload(args, dev)
    checks, moved, drop = check_clustered(w)
    work = w.algorithmic(moved, drop)
    m = time_steps(w, steps, 1)
    floor = roof(work["bytes_compact"])
    res = {"workload": f"1 sequence x {w.S} tokens x {w.L} layers, Hkv 8, head_dim 128, block 16, bf16, "
                       f"keep mask of alternating runs (kept Geom(mean 32), dropped Geom(mean 128)): "
                       f"{int(w.keep_host.sum())} kept; PagedKVCache.compact",
           "step_us": round(m["step_us"], 1), "step_us_median": round(m["step_us_median"], 1),
           "evict_us_per_layer": round(m["step_us"] / w.L, 2), "algorithmic": work,
           "GBps": round(work["bytes_compact"] / (m["step_us"] * 1e-6) / 1e9, 1),
           "pct_of_hbm_peak": round(100 * work["bytes_compact"] / (m["step_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 2),
           "bound": "hbm", "floor_us": round(floor, 1), "frac_of_floor": round(floor / m["step_us"], 4),
           "moved_rows": moved, "blocks_freed": drop, "checks": checks}
    if cpu:
        res["cpu_baseline"] = cpu_clustered(w, work["bytes_compact"])
    del w
    return res


def cpu_runs(w, runs=3):
    """The oracle's reference-style torch CPU path over one whole layer of `w` (layer 0), `runs`
    times from the same inputs: all N action-query folds, one query per fold as the reference
    (lse_attn.py:63-78), then the keep mask, the compaction plan, the row moves of the layer's
    K/V planes and the allocator update (paged.py:141-157).  Seconds per run: (folds, evict)."""
    import torch
    from oracle import reference as ref

    torch.set_num_threads(os.cpu_count() or 1)
    table = [w.host0[1][0]]
    kv_l = w.kv0[0].cpu()
    q = w.q[0, 0].cpu()            # [N, Hq, D]
    lse = w.lse[0, 0].cpu()        # [N, Hq]
    times = []
    for _ in range(runs):
        out = torch.zeros(1, w.hkv, w.width)
        ns = torch.zeros(1, dtype=torch.int32)
        model = ref.PagedCacheModel(w.nb, w.bs, w.hkv, w.d, 1)
        model.kv = kv_l.unsqueeze(0).view(torch.int16).numpy().copy()
        model.free, model.tables, model.seq_used = list(w.host0[0]), {0: list(table[0])}, {0: w.S}
        t0 = time.perf_counter()
        for n in range(w.N):
            ref.action_scores_fold(q[n:n + 1], kv_l, table, [w.S], lse[n:n + 1], out, ns)
        t1 = time.perf_counter()
        model.evict(0, out, w.budget, protected=w.args.sinks)
        t2 = time.perf_counter()
        times.append((t1 - t0, t2 - t1))
    return times


def cpu_ragged(w, nbytes, runs=3):
    """CPU baseline of the ragged batch: the oracle's reference-style path on one layer of the
    request with the least scoring work -- its N action-query folds one query at a time
    (lse_attn.py:63-78), then its evict on that layer (keep mask, plan, row moves, allocator;
    paged.py:141-157) -- `runs` times, median.  The whole step is extrapolated linearly: the
    folds by sum_r N_r S_r over this request's N S, the evict by sum_r S_r over its S, each
    times L layers (a full run would take tens of minutes)."""
    import torch
    from oracle import reference as ref

    torch.set_num_threads(os.cpu_count() or 1)
    s = min(w.reqs, key=lambda r: w.S[r] * w.Nq[r])
    S, N = w.S[s], w.Nq[s]
    table = [w.host0[1][s]]
    kv_l = w.kv0[0].cpu()
    q = w.q[0, s, :N].cpu()
    lse = w.lse[0, s, :N].cpu()
    folds, evicts = [], []
    for _ in range(runs):
        out = torch.zeros(1, w.hkv, w.width)
        ns = torch.zeros(1, dtype=torch.int32)
        model = ref.PagedCacheModel(w.nb, w.bs, w.hkv, w.d, 1)
        model.kv = kv_l.unsqueeze(0).view(torch.int16).numpy().copy()
        model.free, model.tables, model.seq_used = list(w.host0[0]), {0: list(table[0])}, {0: S}
        t0 = time.perf_counter()
        for n in range(N):
            ref.action_scores_fold(q[n:n + 1], kv_l, table, [S], lse[n:n + 1], out, ns)
        t1 = time.perf_counter()
        model.evict(0, out, w.budgets[s], protected=w.sinks)
        t2 = time.perf_counter()
        folds.append(t1 - t0)
        evicts.append(t2 - t1)
        del model
    f_med, e_med = statistics.median(folds), statistics.median(evicts)
    f_scale = sum(n * t for n, t in zip(w.Nq, w.S)) / (N * S) * w.L
    e_scale = sum(w.S) / S * w.L
    step_s = f_med * f_scale + e_med * e_scale
    sample = (f"one layer of request {s} ({S} tokens, {N} action queries): all folds (one action query per "
              f"reference fold) + evict of that layer, {runs} runs, median folds {f_med:.2f} s (runs "
              f"{', '.join(f'{x:.2f}' for x in folds)} s), evict {e_med:.3f} s; extrapolated linearly to the whole "
              f"step: folds x {f_scale:.1f} (sum of N_r S_r over this request's, times {w.L} layers), evict x "
              f"{e_scale:.1f} (sum of S_r over this request's, times {w.L} layers) = {step_s:.0f} s")
    return {"value": round(nbytes / step_s / 1e9, 5), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port", "sample": sample, "runs": runs, "extrapolated": True, "step_s": round(step_s, 1),
            **cpu_info()}


def cpu_clustered(w, nbytes, runs=3):
    """CPU baseline of the 131k compaction: the oracle's reference-style compact (plan_compaction,
    apply_copies on the layer's K and V planes, allocator; paged.py:125-139) on one layer,
    `runs` times, median; the plan is per sequence, so the step is extrapolated as the plan's
    time plus the moves' time times L layers (labelled)."""
    import torch
    from oracle import reference as ref

    torch.set_num_threads(os.cpu_count() or 1)
    kv_l = w.kv0[0].cpu()
    keep = w.keep_host.numpy()
    table = list(w.host0[1][0])
    plans, compacts = [], []
    for _ in range(runs):
        model = ref.PagedCacheModel(w.nb, w.bs, w.hkv, w.d, 1)
        model.kv = kv_l.unsqueeze(0).view(torch.int16).numpy().copy()
        model.free, model.tables, model.seq_used = list(w.host0[0]), {0: list(table)}, {0: w.S}
        t0 = time.perf_counter()
        ref.plan_compaction(keep, w.S, table, w.bs)
        t1 = time.perf_counter()
        model.compact(0, keep)
        t2 = time.perf_counter()
        plans.append(t1 - t0)
        compacts.append(t2 - t1)
        del model
    p_med, c_med = statistics.median(plans), statistics.median(compacts)
    moves = max(c_med - p_med, 0.0)
    step_s = p_med + moves * w.L
    sample = (f"compact of one layer ({w.S} tokens, K and V planes), {runs} runs, median {c_med:.2f} s (runs "
              f"{', '.join(f'{x:.2f}' for x in compacts)} s), of which the plan {p_med:.2f} s; extrapolated "
              f"linearly: plan + moves x {w.L} layers = {step_s:.1f} s")
    return {"value": round(nbytes / step_s / 1e9, 4), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port", "sample": sample, "runs": runs, "extrapolated": True, "step_s": round(step_s, 2),
            **cpu_info()}


def cpu_summary(times, nbytes, what, layers=1):
    """CPU baseline entry from per-run (folds, evict) seconds of one layer: the median run,
    scaled linearly to `layers` layers when that is more than one (labelled)."""
    import torch
    run_s = sorted(f + e for f, e in times)
    med = statistics.median(run_s)
    step_s = med * layers
    sample = (f"{what}: all folds (one action query per reference fold) + keep mask + compaction of one "
              f"layer, {len(times)} runs, median {med:.2f} s (runs {', '.join(f'{x:.2f}' for x in run_s)} s)")
    if layers > 1:
        sample += f"; extrapolated linearly to {layers} layers ({step_s:.0f} s)"
    info = cpu_info()
    return {"value": round(nbytes / step_s / 1e9, 4), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port", "sample": sample, "runs": len(times), "median_s_per_layer": round(med, 3),
            "extrapolated": layers > 1, "step_s": round(step_s, 2), **info}


def cpu_info():
    """The host CPU: /proc/cpuinfo's model name and lscpu's full description."""
    import shutil
    import subprocess
    info = {"cpu_model": cpu_model(), "os_cpu_count": os.cpu_count()}
    if shutil.which("lscpu"):
        try:
            out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        except (OSError, subprocess.SubprocessError):
            out = ""
        keys = {"Model name": "lscpu_model_name", "BIOS Model name": "lscpu_bios_model_name",
                "Socket(s)": "lscpu_sockets", "Core(s) per socket": "lscpu_cores_per_socket",
                "Thread(s) per core": "lscpu_threads_per_core", "CPU(s)": "lscpu_cpus"}
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in keys:
                info[keys[k.strip()]] = v.strip()
    return info


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def score_source_sha():
    """sha256 of the scoring kernel's source: a stored counter figure is used only for the
    kernel it was measured on."""
    import hashlib
    with open(os.path.join(ROOT, "actkv-open_amd", "csrc", "score.hip"), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def load_traffic(path):
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def run_attn(args, dev):
    """Paged attention with the LSE by-product on the main workload's cache shape.

    - queries: 128 action queries per request attending to the whole 32k-token request, every
      layer in one call (the lse producer of the scoring step), then the same with causal limits
      (query n sees the first S - 127 + n tokens);
    - decode: one query per request for a batch of 8 requests of 4k..32k tokens, every layer.
    Time per call from HIP events around back-to-back calls on the launch stream; FLOPs are
    4 * N * Hq * S * D per layer (q.k and p.v), bytes are the K and V rows read."""
    import torch
    from actkv.kernels.lse_attn import paged_decode_attention, paged_decode_attention_ref
    from actkv.paged import PagedKVCache

    L, hq, hkv, d, bs = args.layers, args.q_heads, args.kv_heads, args.head_dim, args.block_size
    gdev = torch.Generator(device=dev).manual_seed(args.seed)

    def make_cache(lens):
        nb = sum(-(-n // bs) for n in lens) + 16
        cache = PagedKVCache(nb, bs, hkv, d, n_layers=L, dtype=torch.bfloat16, device=dev)
        cache.free = torch.randperm(nb, generator=torch.Generator().manual_seed(args.seed)).tolist()
        for r, n in enumerate(lens):
            cache._ensure(r, n)
            cache.seq_used[r] = n
        cache.kv.normal_(generator=gdev)
        return cache

    def timed(fn, reps):
        fn()
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(reps):
            fn()
        ev1.record()
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) * 1e3 / reps

    res = {"metric": "paged attention with lse (the lse producer), time per call", "unit": "us",
           "n_gpus": 1, "higher_is_better": False, "dtype": "bf16", "data": "synthetic"}
    # 128 queries x 32k tokens, all layers
    S, N = args.seq, args.queries
    cache = make_cache([S])
    seq, bt = cache._device_tables([0])
    q = torch.randn(L, 1, N, hq, d, generator=gdev, device=dev, dtype=torch.bfloat16)
    kv_len = torch.arange(S - N + 1, S + 1, device=dev, dtype=torch.int32).view(1, N)
    flops = 4.0 * N * hq * S * d * L
    rows = {}
    for name, kl in (("queries", None), ("queries_causal", kv_len)):
        us = timed(lambda: paged_decode_attention(q, cache.kv, bt, seq, kv_len=kl), max(args.steps // 4, 3))
        rows[name] = {"us": round(us, 1), "TFLOPs": round(flops / (us * 1e-6) / 1e12, 1),
                      "frac_of_bf16_peak": round(flops / (us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4)}
        log(f"attention {name}: {us:.1f} us, {rows[name]['TFLOPs']} TFLOP/s")
    res["queries"] = {"workload": f"{L} layers x 1 request x {S} tokens, {N} queries, Hq {hq} / Hkv {hkv}, "
                                  f"head_dim {d}, block {bs}, bf16", **rows["queries"],
                      "causal": rows["queries_causal"]}
    del cache, q
    torch.cuda.empty_cache()
    # decode: batch 8, one query each
    lens = [int(x) for x in np.random.default_rng(args.seed).integers(4096, 32769, 8)]
    cache = make_cache(lens)
    reqs = list(range(8))
    seq, bt = cache._device_tables(reqs)
    q1 = torch.randn(L, 8, 1, hq, d, generator=gdev, device=dev, dtype=torch.bfloat16)
    us = timed(lambda: paged_decode_attention(q1, cache.kv, bt, seq), max(args.steps, 5))
    nbytes = 2.0 * sum(lens) * hkv * d * 2 * L
    dec = {"workload": f"{L} layers x 8 requests ({min(lens)}..{max(lens)} tokens), 1 query each, bf16",
           "us": round(us, 1), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
           "frac_of_hbm_peak": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    # the reference's stand-in (torch gather + einsum, lse_attn.py:42-60) on the same GPU, one layer
    q0 = q1[0, :, 0].contiguous()
    t_ref = timed(lambda: paged_decode_attention_ref(q0, cache.kv[0], bt, seq), 3)
    t_one = timed(lambda: paged_decode_attention(q0, cache.kv[0], bt, seq), 10)
    dec["one_layer_us"] = round(t_one, 1)
    dec["torch_reference_one_layer_us"] = round(t_ref, 1)
    res["decode"] = dec
    del cache, q1, q0
    torch.cuda.empty_cache()
    res["decode_per_layer"] = decode_per_layer(torch, dev, args, make_cache, timed)
    res["value"] = rows["queries"]["us"]
    res["config"] = {"workload": res["queries"]["workload"], "parallelism": "single-gpu"}
    res.update(run_info(torch, dev))
    line = json.dumps(res)
    print(line)
    if args.out:
        with open(args.out, "w") as f:
            f.write(line + "\n")
    return 0


def decode_per_layer(torch, dev, args, make_cache, timed):
    """A serving decode step's attention: batch 4, one query per request, 4400 tokens each,
    one call per layer (the cache pointer at the layer) for all layers, captured in a HIP graph
    as a served decode step is.  Tables 4400 tokens wide, and 8400 wide (a session sized for
    8400 tokens whose requests hold 4400 after a compaction).  Bytes: the K and V rows read."""
    from actkv.kernels.lse_attn import paged_decode_attention
    L, hq, hkv, d, bs = args.layers, args.q_heads, args.kv_heads, args.head_dim, args.block_size
    B, S = 4, 4400
    cache = make_cache([S] * B)
    reqs = list(range(B))
    seq, bt = cache._device_tables(reqs)
    q = torch.randn(L, B, hq, d, device=dev, dtype=torch.bfloat16)
    nbytes = 2.0 * B * S * hkv * d * 2 * L
    out = {"workload": f"{L} layers x {B} requests x {S} tokens, one query each, one call per layer, "
                       f"replayed from a HIP graph, bf16"}
    for name, width in (("table_4400", -(-S // bs)), ("table_8400", -(-8400 // bs))):
        wide = torch.zeros(B, width, dtype=torch.int32, device=dev)
        wide[:, : bt.shape[1]] = bt
        run = lambda: [paged_decode_attention(q[l], cache.kv[l], wide, seq) for l in range(L)]
        run()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            run()
        us = timed(g.replay, max(args.steps, 10)) / L
        out[name] = {"us_per_layer": round(us, 2), "GBps": round(nbytes / L / (us * 1e-6) / 1e9, 1),
                     "frac_of_hbm_peak": round(nbytes / L / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"decode per layer, {name}: {us:.2f} us, {out[name]['GBps']} GB/s")
    return out


def _append_summary(per_round, L, hkv, d):
    """Append launches of the agent loop: bf16 source rows read and cache rows written, K and
    V planes of every layer (algorithmic bytes 2 planes x 2 (read + write) x L x Hkv x D x 2 B
    per token)."""
    us = [p["append_us"] for p in per_round]
    gbs = [p["appended"] * 2 * 2 * L * hkv * d * 2 / (p["append_us"] * 1e-6) / 1e9 for p in per_round]
    return {"tokens_per_round_median": int(statistics.median(p["appended"] for p in per_round)),
            "us_median": round(statistics.median(us), 1),
            "GBps_median": round(statistics.median(gbs), 1),
            "pct_of_hbm_peak": round(100 * statistics.median(gbs) / HBM_PEAK_GBS, 1),
            "host_us_median": round(statistics.median(p["append_host_us"] for p in per_round), 1)}


def run_ora(args, dev):
    """The agent-loop workload on its own (bench.py --ora): prints its JSON line."""
    result = ora_rounds(args, dev, args.ora_rounds, per_round=True)
    line = json.dumps(result)
    print(line)
    if args.out:
        with open(args.out, "w") as f:
            f.write(line + "\n")
    return 0


def ora_rounds(args, dev, rounds, per_round=False):
    """Agent-loop workload: 50 rounds on a Qwen3-8B-shaped 36-layer cache holding 4 sequences.
    Each round appends, per sequence, U[512, 2048] observation + U[128, 512] reasoning +
    U[32, 64] action tokens (bf16 K/V ~ N(0,1), seeded; one batched append launch, timed on
    its own and reported beside the eviction), scores the action tokens against the
    cache with causal limits (action token j sees the prefix and action tokens <= j; their lse
    comes from the paged attention kernel, untimed, as from the model's forward pass), updates
    the LRFU keep scores (decay 0.5, top-p 0.9), keeps 4 sinks plus the top
    `budget` tokens by the layer-average keep score (budget rising linearly 4096 -> 16384) and
    compacts.  Timed per round with HIP events: scoring + LRFU update + keep + compaction."""
    import torch
    from actkv.kernels.lrfu import LRFUConfig, PagedLRFU
    from actkv.paged import PagedKVCache

    L, hq, hkv, d, bs, R = args.layers, args.q_heads, args.kv_heads, args.head_dim, args.block_size, 4
    b_lo, b_hi, sinks = 4096, 16384, 4
    cap = ((b_hi + sinks + 2048 + 512 + 64 + bs - 1) // bs) * bs
    nb = R * (cap // bs + 2) + 64
    gcpu = torch.Generator().manual_seed(args.seed)
    cache = PagedKVCache(nb, bs, hkv, d, n_layers=L, dtype=torch.bfloat16, device=dev)
    cache.free = torch.randperm(nb, generator=gcpu).tolist()
    gdev = torch.Generator(device=dev).manual_seed(args.seed + 1)
    rng = np.random.default_rng(args.seed)
    reqs = list(range(R))
    lr = PagedLRFU(cache, reqs, cap, LRFUConfig(decay=0.5, top_p=0.9))
    scale = d ** -0.5
    per_round = []
    # Python's collector: a full collection walks every tracked object of the process
    # (torch's import alone leaves hundreds of thousands) and stalls the host for tens of
    # milliseconds when it lands inside a round; time spent collecting is recorded per round
    gc_ms = [0.0, 0.0]

    def _gc_clock(phase, info):
        if phase == "start":
            gc_ms[1] = time.perf_counter()
        else:
            gc_ms[0] += (time.perf_counter() - gc_ms[1]) * 1e3

    gc.callbacks.append(_gc_clock)
    if not args.no_gc_freeze:
        gc.collect()
        gc.freeze()
    log(f"agent loop: {rounds} rounds, {R} sequences, {L} layers")
    schedule = max(args.ora_rounds, rounds)
    for rnd in range(rounds):
        budget = int(round(b_lo + (b_hi - b_lo) * rnd / max(schedule - 1, 1)))
        n_act, counts = [], []
        for r in reqs:
            n_new = int(rng.integers(512, 2049)) + int(rng.integers(128, 513))
            a = int(rng.integers(32, 65))
            n_act.append(a)
            counts.append(n_new + a)
        k = torch.randn(L, sum(counts), hkv, d, generator=gdev, device=dev, dtype=torch.bfloat16)
        v = torch.randn(L, sum(counts), hkv, d, generator=gdev, device=dev, dtype=torch.bfloat16)
        torch.cuda.synchronize()
        # the round's new tokens of all sequences, every layer, in one append launch
        ea = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ea[0].record()
        gc_ms[0] = 0.0
        ha0 = time.perf_counter()
        cache.append_batch(reqs, k, v, counts)
        ha1 = time.perf_counter()
        gc_append = gc_ms[0]
        ea[1].record()
        del k, v
        nmax = max(n_act)
        q = torch.randn(L, R, nmax, hq, d, generator=gdev, device=dev, dtype=torch.bfloat16)
        kv_len = torch.zeros(R, nmax, dtype=torch.int32, device=dev)
        for j, r in enumerate(reqs):
            S = cache.seq_used[r]
            kv_len[j, : n_act[j]] = torch.arange(S - n_act[j] + 1, S + 1, device=dev, dtype=torch.int32)
        n_valid = torch.tensor(n_act, dtype=torch.int32, device=dev)
        # the action tokens' attention and its lse (causal), as the model's forward pass
        # produces them; outside the timed region
        _, lse = cache.decode_attention(reqs, q, layer=None, scale=scale, n_valid=n_valid, kv_len=kv_len)
        tokens_before = sum(cache.seq_used[r] for r in reqs)
        free_before = len(cache.free)
        lr.begin_round()
        torch.cuda.synchronize()
        # one interval per round: an event between the two calls resolves before the scoring
        # kernel ends on this runtime, so the round is not split
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record()
        gc_ms[0] = 0.0
        h0 = time.perf_counter()
        cache.cal_attn(reqs, q, lse, lr.scores, lr.n_seen, layer=None, n_valid=n_valid, kv_len=kv_len)
        lr.evict(budget, protected=sinks, n_action=n_act)
        h1 = time.perf_counter()
        gc_round = gc_ms[0]
        ev[1].record()
        torch.cuda.synchronize()
        per_round.append({"round": rnd, "budget": budget, "tokens_before": tokens_before,
                          "tokens_after": sum(cache.seq_used[r] for r in reqs),
                          "blocks_reclaimed": len(cache.free) - free_before,
                          "evict_us": ev[0].elapsed_time(ev[1]) * 1e3,
                          "host_us": (h1 - h0) * 1e6,
                          "gc_us": gc_round * 1e3,
                          "appended": sum(counts),
                          "append_us": ea[0].elapsed_time(ea[1]) * 1e3,
                          "append_host_us": (ha1 - ha0) * 1e6,
                          "append_gc_us": gc_append * 1e3})
        if rnd % 10 == 0 or rnd == rounds - 1:
            pr = per_round[-1]
            log(f"round {rnd}: {pr['tokens_before']} -> {pr['tokens_after']} tokens, "
                f"{pr['blocks_reclaimed']} blocks reclaimed, {pr['evict_us']:.0f} us")
    lat = sorted(p["evict_us"] for p in per_round)
    result = {
        "metric": "agent-loop evict latency per round (score action region + LRFU keep + compact)",
        "value": round(statistics.median(lat), 1), "unit": "us", "n_gpus": 1, "rounds": rounds,
        "higher_is_better": False, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"agent loop: {rounds} rounds, batch {R}, {L} layers, Hq {hq} / Hkv {hkv}, "
                               f"head_dim {d}, block {bs}, bf16; per round per sequence U[512,2048] obs + "
                               f"U[128,512] reasoning + U[32,64] action tokens; LRFU decay 0.5 top-p 0.9; "
                               f"budget {b_lo}->{b_hi} + {sinks} sinks", "parallelism": "single-gpu"},
        "evict_us": {"mean": round(statistics.mean(lat), 1), "median": round(statistics.median(lat), 1),
                     "p90": round(lat[int(0.9 * (len(lat) - 1))], 1), "max": round(lat[-1], 1)},
        "evict_us_per_layer_median": round(statistics.median(lat) / L, 2),
        "append": _append_summary(per_round, L, hkv, d),
        "gc_frozen": not args.no_gc_freeze,
        "gc_us_max": round(max(p["gc_us"] for p in per_round), 1),
        "blocks_reclaimed_total": sum(p["blocks_reclaimed"] for p in per_round),
    }
    if per_round:
        result["per_round"] = [{k: (round(v, 1) if isinstance(v, float) else v) for k, v in p.items()}
                               for p in per_round]
        result.update(run_info(torch, dev))
    del cache, lr
    torch.cuda.empty_cache()
    return result


def run_serve(args, dev):
    """Serving on the paged cache: a Qwen3-8B-shaped transformers model (36 layers, hidden 4096,
    Hq 32 / Hkv 8, head_dim 128, MLP 12288, vocab 151936; random bf16 weights, no checkpoint)
    runs through PagedSession: the attention of every layer is the paged HIP kernel, new K/V
    go in with the append kernel.  A batch of sequences prefills a prompt (the first 256 tokens
    protected), then runs rounds of greedy decode steps whose last tokens are the action region;
    each round ends with ActKV's compression (scoring of the action tokens from their lse, LRFU
    update, keep, compaction) to the budget.  Reports prefill and decode throughput and the
    end-of-round latency."""
    import torch
    from transformers import Qwen3Config, Qwen3ForCausalLM
    from actkv.hf import PagedSession

    B, P = args.serve_batch, args.serve_prompt
    rounds, steps, n_act, budget = args.serve_rounds, args.serve_steps, args.serve_action, args.serve_budget
    cfg = Qwen3Config(vocab_size=151936, hidden_size=4096, intermediate_size=12288, num_hidden_layers=36,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=128, max_position_embeddings=65536,
                      rope_theta=1000000.0, tie_word_embeddings=False)
    log(f"building a random-weight Qwen3-8B-shaped model (bf16)")
    torch.manual_seed(args.seed)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            model = Qwen3ForCausalLM(cfg).eval()
    finally:
        torch.set_default_dtype(prev)
    n_params = sum(p.numel() for p in model.parameters())
    max_tokens = P + rounds * steps + 64
    sess = PagedSession(model, B, max_tokens=max_tokens, block_size=args.block_size, graph=not args.serve_eager)
    g = torch.Generator(device=dev).manual_seed(args.seed + 1)
    prompt = torch.randint(0, cfg.vocab_size, (B, P), generator=g, device=dev)
    gc.collect()
    gc.freeze()
    torch.cuda.synchronize()
    log(f"prefill {B} x {P} tokens ({n_params / 1e9:.2f}B parameters)")
    t0 = time.perf_counter()
    sess.prefill(prompt[:, :256], protected=True)
    logits = sess.prefill(prompt[:, 256:])
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    tok = logits.argmax(-1)
    per_round = []
    for rnd in range(rounds):
        sess.begin_round()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for j in range(steps):
            logits = sess.decode(tok, in_action=j >= steps - n_act)
            tok = logits.argmax(-1)
        torch.cuda.synchronize()
        dec_s = time.perf_counter() - t0
        before = [sess.kv.seq_used[r] for r in sess.reqs]
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record()
        h0 = time.perf_counter()
        sess.end_round(budget)
        h1 = time.perf_counter()
        ev[1].record()
        torch.cuda.synchronize()
        per_round.append({"round": rnd, "tokens_before": before[0], "tokens_after": sess.kv.seq_used[0],
                          "decode_ms_per_step": dec_s / steps * 1e3,
                          "decode_tokens_per_s": B * steps / dec_s,
                          "end_round_us": ev[0].elapsed_time(ev[1]) * 1e3, "end_round_host_us": (h1 - h0) * 1e6})
        pr = per_round[-1]
        log(f"round {rnd}: {pr['tokens_before']} -> {pr['tokens_after']} tokens per sequence, decode "
            f"{pr['decode_ms_per_step']:.1f} ms/step, end of round {pr['end_round_us']:.0f} us")
    dec = [p["decode_tokens_per_s"] for p in per_round]
    result = {
        "metric": "serving on the paged cache: decode tokens/s with ActKV compression each round",
        "value": round(statistics.median(dec), 1), "unit": "tokens/s", "n_gpus": 1,
        "higher_is_better": True, "dtype": "bf16", "data": "synthetic (random weights, random prompt ids)",
        "config": {"workload": f"Qwen3-8B-shaped transformers model ({n_params / 1e9:.2f}B parameters, random "
                               f"bf16 weights), batch {B}, prompt {P} (256 protected), {rounds} rounds x {steps} "
                               f"greedy decode steps, last {n_act} of each round scored as the action region, "
                               f"budget {budget}, LRFU decay 0.5 top-p 0.9, block {args.block_size}",
                   "parallelism": "single-gpu"},
        "decode_launch": "python (eager)" if args.serve_eager else "hip graph replay",
        "prefill_tokens_per_s": round(B * P / prefill_s, 1),
        "decode_ms_per_step_median": round(statistics.median(p["decode_ms_per_step"] for p in per_round), 2),
        "end_round_us_median": round(statistics.median(p["end_round_us"] for p in per_round), 1),
        "per_round": [{k: (round(v, 1) if isinstance(v, float) else v) for k, v in p.items()} for p in per_round],
        **run_info(torch, dev),
    }
    line = json.dumps(result)
    print(line)
    if args.out:
        with open(args.out, "w") as f:
            f.write(line + "\n")
    return 0


def main(argv=None):
    args = parse(argv)
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported (one GPU only: the "
              "eviction path shards by request or by KV head), run with --gpus 1", file=sys.stderr)
        return 2
    import torch
    from actkv import _hip

    if not _hip.available():
        print("bench.py needs a ROCm GPU and the built libactkv_hip.so", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.ora:
        return run_ora(args, dev)
    if args.attn:
        return run_attn(args, dev)
    if args.serve:
        return run_serve(args, dev)
    if args.configs_only:
        configs = {"cfg1": run_cfg1(args, dev, cpu=False), "cfg3": run_cfg3(args, dev), "cfg4": run_cfg4(args, dev)}
        line = json.dumps({"configs": configs, **run_info(torch, dev)})
        print(line)
        if args.out:
            with open(args.out, "w") as f:
                f.write(line + "\n")
        return 0

    log(f"building the {args.layers}-layer workload")
    w = Workload(args, args.layers, dev)
    # a full collection walks every tracked object of the process (torch's import alone leaves
    # hundreds of thousands) and stalls the host for tens of milliseconds; the startup heap is
    # frozen after setup, as a serving process does after loading
    gc.collect()
    gc.freeze()
    log("checking one step against the oracle")
    checks, moved, drop = check_step(w)
    log(f"checks {checks}; timing {args.warmup} + {args.steps} steps")
    work = w.algorithmic(moved, drop)
    m = measure(w, args.steps, args.warmup)
    k_us = m["score_us"]
    total_bytes = work["bytes_score"] + work["bytes_keep"] + work["bytes_compact"]
    gbs = total_bytes / (m["step_us"] * 1e-6) / 1e9
    score_tflops = work["flops_score"] / (k_us * 1e-6) / 1e12
    traffic = load_traffic(args.traffic)
    traffic_bytes = None
    if traffic and traffic.get("layers") == args.layers and traffic.get("seq") == args.seq \
            and traffic.get("queries") == args.queries and traffic.get("score_hip_sha256") == score_source_sha():
        traffic_bytes = traffic.get("hbm_bytes_per_launch")

    log(f"step {m['step_us']:.1f} us (synchronised launches {m['step_us_sync']:.1f} us), scoring call {k_us:.1f} us")
    extra_mb = extra_memory_mb(w)
    power = None
    if not args.no_power:
        log("power and clock while scoring")
        power = power_leg(w)
    ceiling = None
    if power:
        # the step's floor at the clock the scoring call actually runs at (the board's power
        # limit): scoring at the dense bf16 peak scaled to that clock (or its bytes at 8 TB/s,
        # whichever is longer), keep mask and compaction at 8 TB/s
        clk = power["gfx_clock_mhz"]
        f_score = max(work["flops_score"] / (BF16_PEAK_TFLOPS * 1e12 * clk / 2400.0),
                      work["bytes_score"] / (HBM_PEAK_GBS * 1e9))
        floor_us = (f_score + (work["bytes_keep"] + work["bytes_compact"]) / (HBM_PEAK_GBS * 1e9)) * 1e6
        ceil_gbs = total_bytes / (floor_us * 1e-6) / 1e9
        ceiling = {"gfx_clock_mhz": clk, "step_floor_us": round(floor_us, 1), "GBps": round(ceil_gbs, 1),
                   "pct_of_hbm_peak": round(100 * ceil_gbs / HBM_PEAK_GBS, 2),
                   "value_frac_of_ceiling": round(gbs / ceil_gbs, 4),
                   "basis": "scoring flops at the dense bf16 peak scaled to the measured GFX clock, keep "
                            "mask and compaction bytes at 8 TB/s"}
    single = None
    cpu = None
    if args.layers != 1 and not (args.no_single_layer and args.no_cpu):
        log("one-layer workload")
        w1 = Workload(args, 1, dev)
        if not args.no_single_layer:
            c1, mv1, dr1 = check_step(w1)
            wk1 = w1.algorithmic(mv1, dr1)
            m1 = measure(w1, args.steps, args.warmup)
            b1 = wk1["bytes_score"] + wk1["bytes_keep"] + wk1["bytes_compact"]
            single = {"step_us": round(m1["step_us"], 2), "score_us": round(m1["score_us"], 2),
                      "evict_us": round(m1["evict_us"], 2),
                      "score_compact_GBps": round(b1 / (m1["step_us"] * 1e-6) / 1e9, 1),
                      "pct_of_hbm_peak": round(100 * b1 / (m1["step_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 2),
                      "score_TFLOPs": round(wk1["flops_score"] / (m1["score_us"] * 1e-6) / 1e12, 1),
                      "checks": c1}
        if not args.no_cpu:
            # the one-layer case in full, on this host's cores: the baseline of the one-layer
            # workload as it is, and of the whole step extrapolated linearly in layers
            log(f"CPU baseline: the {args.seq}-token layer in full, {args.cpu_runs} runs")
            times = cpu_runs(w1, args.cpu_runs)
            what = f"one {args.seq}-token layer with {args.queries} action queries in full"
            cpu = cpu_summary(times, total_bytes, what, layers=args.layers)
            if single is not None:
                single["cpu_baseline"] = cpu_summary(times, b1, what)
        del w1

    log("apply_copies on a plan of the compaction's size")
    copies = time_apply_copies(torch, w, moved, max(args.steps, 5))  # rewrites rows: after every other leg
    del w
    torch.cuda.empty_cache()
    table1 = None
    if not args.no_table1:
        log("the reference bench's Table-1 cases")
        table1 = run_table1(torch, dev, seed=args.seed)
    configs = None
    if not args.no_configs:
        configs = {}
        log("leg cfg1: one fp16 layer of 2048 tokens, 64 action queries")
        configs["cfg1"] = run_cfg1(args, dev, cpu=not args.no_cpu)
        torch.cuda.empty_cache()
        log("leg cfg3: 36 layers x 8 ragged sequences, one evict_batch")
        configs["cfg3"] = run_cfg3(args, dev, cpu=not args.no_cpu)
        torch.cuda.empty_cache()
        log("leg cfg4: 131072 tokens x 36 layers, clustered keep, compaction")
        configs["cfg4"] = run_cfg4(args, dev, cpu=not args.no_cpu)
        torch.cuda.empty_cache()
    ora = None
    if args.ora_short > 0 and args.layers == 36:
        log(f"agent loop, first {args.ora_short} rounds")
        ora = ora_rounds(args, dev, args.ora_short)
        ora = {k: ora[k] for k in ("config", "rounds", "evict_us", "evict_us_per_layer_median", "append",
                                   "blocks_reclaimed_total", "gc_us_max")}

    result = {
        "metric": "score+compact HBM GB/s (% of 8 TB/s) and evict us/layer, Qwen3-8B shape 32k",
        "value": round(gbs, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(m["step_us"] / 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"qwen3-8b-shaped paged cache: {args.layers} layers x 1 sequence x {args.seq} "
                               f"tokens, Hq {args.q_heads} / Hkv {args.kv_heads}, head_dim {args.head_dim}, "
                               f"block {args.block_size}, bf16, {args.queries} action queries, keep "
                               f"{args.keep:.0%} + {args.sinks} sinks, shuffled blocks",
                   "layers": args.layers, "seq_len": args.seq, "action_queries": args.queries,
                   "parallelism": "single-gpu"},
        "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "evict_us_per_layer": round(m["step_us"] / args.layers, 3),
        "phases_us": {"score": round(m["score_us"], 2), "keep_mask+compact": round(m["evict_us"], 2),
                      "step_median": round(m["step_us_median"], 2),
                      "step_with_host_launch_exposed": round(m["step_us_sync"], 2)},
        "algorithmic": work,
        "roofline": {"kernel": "score_qreg_kernel (actkv_action_scores)", "bound": "mfma",
                     "achieved": round(score_tflops, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(score_tflops / BF16_PEAK_TFLOPS, 4), "traffic": traffic_bytes,
                     "launch_us": round(k_us, 2),
                     "hbm_GBps_algorithmic": round(work["bytes_score"] / (k_us * 1e-6) / 1e9, 1),
                     "ceiling_at_clock": ceiling},
        "cpu_baseline": cpu,
        "single_layer": single,
        "configs": configs,
        "apply_copies": copies,
        "extra_mb_per_step": extra_mb,
        "power": power,
        "table1": table1,
        "ora": ora,
        "checks": checks,
        "wall_s_incl_restore": round(m["wall_s_incl_restore"], 3),
        **run_info(torch, dev),
    }
    line = json.dumps(result)
    print(line)
    if args.out:
        with open(args.out, "w") as f:
            f.write(line + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
