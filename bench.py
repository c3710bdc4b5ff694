"""Benchmark of the LongSpark verify-and-refresh hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

A step is one pass of the hot path over one batch of synthetic input that is
already resident in HBM.  W untimed warm-up steps run first, then exactly K
timed steps bracketed by ``torch.cuda.synchronize()``.  Rank 0 prints one
JSON line with the metric (verified rows/s), the roofline of the dominant
kernel (algorithmic bytes / its average duration, measured with HIP events
on the stream it runs on) and a CPU baseline (the oracle's torch-CPU
restatement of the reference path, timed on a bounded sample on this host).

This build targets one GPU; ``--gpus`` above 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from types import SimpleNamespace

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
V = 151936

# HBM bytes per launch of each workload's dominant kernel, from rocprofv3
# FETCH_SIZE and WRITE_SIZE passes scaled by the counters' readings for a 1 GiB
# copy (x2.0 and x1.0).  The commands and raw counter values are in the
# profiles/ summary named beside each figure.
TRAFFIC = {
    "verify_wave_kernel": (712_314_120, "profiles/verify_wave_kernel_verify_sample_B128_K16_V151936.md"),
    "greedy_verify_kernel": (622_640_864, "profiles/greedy_verify_kernel_B128_K16_V151936.md"),
    "window_gather_kernel": (604_552_647, "profiles/window_gather_kernel_B8_L36_Hkv8_D128_ctx131072.md"),
    "summary_kernel": (646_838_203, "profiles/summary_kernel_B8_L36_R256_W16.md"),
    "softmax_temp_resident_kernel": (1_868_715_744, "profiles/softmax_temp_resident_kernel_B128_K16_V151936.md"),
    "chain_kernel": (158_529_676, "profiles/chain_kernel_chain_sampling_B128_K16_V151936.md"),
    "request_bias_kernel": (1_403_662_037, "profiles/request_bias_kernel_adjust_logits_B128_K16_V151936.md"),
    "sample_step_kernel": (156_502_794, "profiles/sample_step_kernel_B128_V151936.md"),
    "draft_attention_kernel": (204_226_688, "profiles/draft_attention_kernel_B128_Hq32_Hkv8_raw256.md"),
    "draft_merge_kernel": (77_205_083, "profiles/draft_merge_kernel_B128_Hq32_Hkv8.md"),
    "prefill_kernel + prefill_combine_kernel": (
        2_759_473_028, "profiles/prefill_kernel_global16_prefill_L5_Hkv8_D128_ctx131072.md"),
}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def time_cpu(fn, *, warmup=3, reps=20, budget_s=30.0):
    """Median wall time (s) of ``fn`` over ``reps`` runs after ``warmup`` runs,
    stopping early once ``budget_s`` of timed work has accumulated (>= 5 runs)."""
    for _ in range(warmup):
        fn()
    times = []
    spent = 0.0
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        dt = time.perf_counter() - t0
        times.append(dt)
        spent += dt
        if spent > budget_s and len(times) >= 5:
            break
    return statistics.median(times), len(times)


# --------------------------------------------------------------------------
# workloads
# --------------------------------------------------------------------------

class GreedyVerify:
    """Greedy chain verification, batch 128 x block 16 x vocab 151,936 bf16."""

    copies, rotate = 2, ("logits", "cand")

    name = "verify_greedy"

    def __init__(self, dev, batch=128, width=16, vocab=V):
        from longspark_amd import workloads
        self.dev, self.batch, self.width, self.vocab = dev, batch, width, vocab
        self.logits, self.cand = workloads.greedy_inputs(batch, width, vocab, seed=2024, device=dev,
                                                         gen_device=dev)
        self.rows = batch * width
        # algorithmic bytes: every logit once, candidates once, outputs once
        self.bytes = self.rows * vocab * 2 + batch * width * 4 + batch * (4 + 8)
        self.kernel = "greedy_verify_kernel"

    def step(self):
        from longspark_amd import verify
        return verify.verify_greedy(logits=self.logits, candidates=self.cand, width=self.width)

    def config(self):
        return {"workload": f"greedy chain verify B={self.batch} K={self.width} V={self.vocab} bf16 "
                            "(logits N(0,3^2), drafted token +8 w.p. 0.7)",
                "batch": self.batch, "block": self.width, "vocab": self.vocab}

    def cpu_baseline(self, threads):
        from oracle import verify as ov
        from longspark_amd import workloads
        b = 16
        logits, cand = workloads.greedy_inputs(b, self.width, self.vocab, seed=7)
        logits = logits.float()  # the reference verifier sees fp32 logits
        cand = cand.long()
        torch.set_num_threads(threads)
        med, n = time_cpu(lambda: ov.accept_greedy(cand, logits, self.width))
        return {"rows_per_s": b * self.width / med, "sample": f"B={b} x K={self.width} x V={self.vocab} "
                f"fp32 logits, median of {n} runs", "threads": threads}


class HipEvents:
    """hipEvent_t handles from the HIP runtime (for timing kernels that one C ABI
    call launches back to back on a stream).  The events are created for timing
    only (hipEventDisableSystemFence): recording one then costs no cache
    writeback, which would otherwise add a gap of several microseconds to the
    stream at every event."""

    DISABLE_SYSTEM_FENCE = 0x20000000

    def __init__(self, n):
        import ctypes
        self.ct = ctypes
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.handles = (ctypes.c_void_p * n)()
        for i in range(n):
            h = ctypes.c_void_p()
            if self.hip.hipEventCreateWithFlags(ctypes.byref(h), self.DISABLE_SYSTEM_FENCE) != 0:
                raise RuntimeError("hipEventCreateWithFlags failed")
            self.handles[i] = h

    def group(self, i, k):
        """ctypes array view of events [i*k, (i+1)*k)."""
        return (self.ct.c_void_p * k).from_address(self.ct.addressof(self.handles) + i * k * self.ct.sizeof(self.ct.c_void_p))

    def elapsed_ms(self, a, b):
        ms = self.ct.c_float()
        if self.hip.hipEventElapsedTime(self.ct.byref(ms), self.handles[a], self.handles[b]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value


class StochasticVerify:
    """Fused stochastic verify, batch 128 x block 16 x vocab 151,936 bf16:
    temperature 0.7, top-k 50, top-p 0.95, repetition 1.05 over a 2048-token
    Zipf(1.1) history; draft rows fp32; one penalty-table build + one fused
    verify per step."""

    copies, rotate = 2, ("d",)

    name = "verify_sample"

    boost_drafted = False

    def __init__(self, dev, batch=128, width=16, vocab=V):
        from longspark_amd import workloads
        self.dev, self.batch, self.width, self.vocab = dev, batch, width, vocab
        self.cfg = dict(workloads.VERIFY_BENCH_CFG)
        self.d = workloads.verify_bench_inputs(dev, batch, width, vocab, boost_drafted=self.boost_drafted)
        self.rows = batch * width
        # The dominant kernel scans every target row and, in the same launch, the
        # fp32 draft row at the rejection of every request that rejects a token.
        self.kernel = "verify_wave_kernel"
        self.kernel_bytes = None                            # set by count_rejected()
        # whole verify, as counted for the workload: logits + one fp32 draft row per
        # request + the int32 history
        self.bytes = self.rows * vocab * 2 + batch * vocab * 4 + batch * self.cfg["history_len"] * 4
        self.events = None
        self.step_idx = 0

    def count_rejected(self, out):
        """Algorithmic bytes of the dominant kernel for this input: every target
        logit once, plus the draft row of each request that rejects."""
        accept = out[0]
        rejected = int((accept < self.width - 1).sum().item())
        self.rejected = rejected
        self.mean_accepted = float(accept.float().mean().item())
        self.kernel_bytes = self.rows * self.vocab * 2 + rejected * self.vocab * 4

    # One timed step in TIMING_EVERY records the four HIP events of the C ABI
    # (before and after the verify_wave kernel, before and after resolve):
    # each recorded event adds a few microseconds of stream time, so timing
    # every step would understate the throughput of the steps themselves.
    TIMING_EVERY = 4

    def arm_timing(self, steps):
        n = (steps + self.TIMING_EVERY - 1) // self.TIMING_EVERY
        self.events = HipEvents(4 * n)
        self.step_idx = 0
        self.timed = 0

    def step(self):
        from longspark_amd import penalties, verify
        d, p = self.d, self.d["params"]
        tables = penalties.build_penalty_tables(d["history"], self.vocab, repetition=d["repetition"])
        ev = None
        if self.events is not None:
            if self.step_idx % self.TIMING_EVERY == 0:
                ev = self.events.group(self.timed, 4)
                self.timed += 1
            self.step_idx += 1
        return verify.verify_sample(
            logits=d["logits"], candidates=d["candidates"], width=self.width, temperatures=p.temperatures,
            top_ks=p.top_ks, top_ps=p.top_ps, min_ps=p.min_ps, max_top_k=50, draft_logits=d["draft_logits"],
            draft_token_probs=d["draft_token_probs"], draft_top_ks=p.top_ks, draft_top_ps=p.top_ps,
            uniforms=d["uniforms"], final_uniforms=d["final_uniforms"], penalties=tables, timing_events=ev,
            scan_hint=1)

    def kernel_times_ms(self):
        n = self.timed
        e = self.events
        scan = sum(e.elapsed_ms(4 * i, 4 * i + 1) for i in range(n)) / n
        between = sum(e.elapsed_ms(4 * i + 1, 4 * i + 2) for i in range(n)) / n
        resolve = sum(e.elapsed_ms(4 * i + 2, 4 * i + 3) for i in range(n)) / n
        return {"verify_wave_kernel": scan, "between (fallback / draft kernels when launched)": between,
                "resolve_kernel": resolve}

    def config(self):
        where = ("+8 on the drafted token with probability 0.7 (applied after drafting)" if self.boost_drafted
                 else "+8 on uniform random candidates (replaced by the tokens drawn from q)")
        return {"workload": f"fused stochastic verify B={self.batch} K={self.width} V={self.vocab} bf16, T 0.7, "
                            "top-k 50, top-p 0.95, repetition 1.05 over a 2048-token Zipf history; draft rows fp32; "
                            f"target boost {where}",
                "batch": self.batch, "block": self.width, "vocab": self.vocab,
                "rejecting_requests": getattr(self, "rejected", None),
                "mean_accepted": getattr(self, "mean_accepted", None)}

    def cpu_baseline(self, threads):
        from oracle import verify as ov
        from longspark_amd import workloads
        b = 2
        d = workloads.stochastic_inputs(b, self.width, self.vocab, seed=7, **self.cfg)
        p = d["params"]
        add, scale = ov.penalty_tables(list(d["history"]), self.vocab, d["repetition"], d["presence"], d["frequency"])
        torch.set_num_threads(threads)

        def run():
            ov.verify_sample(logits=d["logits"], candidates=d["candidates"].long(), draft_logits=d["draft_logits"],
                             draft_token_probs=d["draft_token_probs"], uniforms=d["uniforms"],
                             final_uniforms=d["final_uniforms"], temperatures=p.temperatures, top_ks=p.top_ks,
                             top_ps=p.top_ps, min_ps=p.min_ps, additive=add, scaling=scale,
                             draft_top_ks=p.top_ks, draft_top_ps=p.top_ps, draft_min_ps=p.min_ps)
        med, n = time_cpu(run)
        return {"rows_per_s": b * self.width / med, "threads": threads,
                "sample": f"B={b} x K={self.width} x V={self.vocab} (same sampling config), oracle torch-CPU path "
                          f"(penalties, target distribution, acceptance, residual draw), median of {n} runs"}


class StochasticVerifyHighAccept(StochasticVerify):
    """The fused stochastic verify of ``verify_sample`` with the +8 target
    boost on the drafted tokens (probability 0.7 per position, applied after
    drafting): requests accept long prefixes and reject late, so the draft
    slices wait on later target rows and some requests draw their bonus from
    the last target row."""

    name = "verify_sample_high_accept"
    boost_drafted = True


class WindowGather:
    """Recent-window gather, Qwen3-8B geometry: 36 layers, 8 KV heads, head_dim
    128, page size 16, batch 8 at a 131,072-token context (window 256).

    The pool holds 8 x 131,072 tokens per layer (K and V, 154.6 GB) with the
    pages of every request placed by one random permutation; only the pages
    the window touches are filled (N(0,1) bf16) -- the rest is allocated but
    never read, so filling it would only lengthen the set-up.

    Consecutive steps rotate over ``rotate`` disjoint windows (contexts
    131,072, 130,816, ... one window apart) and as many output views, so one
    rotation reads 4 x 302 MB: more than the 256 MB last-level cache, and no
    step finds the previous step's rows in it."""

    name = "kv_window_gather"
    metric = "recent-window gather GB/s (algorithmic bytes) at 36L x 8 Hkv x D128, ps 16, B 8, ctx 131072"
    unit = "GB/s"

    def __init__(self, dev, batch=8, layers=36, heads=8, dim=128, page_size=16, context=131072, window=256,
                 rotate=4):
        from longspark_amd import workloads
        self.dev, self.batch, self.layers, self.heads, self.dim = dev, batch, layers, heads, dim
        self.page_size, self.context, self.window = page_size, context, window
        w = workloads.window_pool(dev, batch=batch, layers=layers, heads=heads, dim=dim, page_size=page_size,
                                  context=context, window=window, rotate=rotate)
        self.k, self.v, self.table, self.seq_sets = w["k"], w["v"], w["table"], w["seq_sets"]
        self.seq_lens = self.seq_sets[0]
        self.outs = [torch.empty(batch, layers, 2, heads, window, dim, dtype=torch.bfloat16, device=dev)
                     for _ in range(rotate)]
        self.out = self.outs[0]
        self.turn = 0
        self.bytes = 2 * self.out.numel() * 2          # every window row read once and written once
        self.kernel = "window_gather_kernel"
        self.units = self.bytes / 1e9

    def step(self):
        from longspark_amd import kvwindow
        i = self.turn % len(self.outs)
        self.turn += 1
        return kvwindow.gather_window(self.k, self.v, self.table, self.seq_sets[i], page_size=self.page_size,
                                      window=self.window, out=self.outs[i])

    def config(self):
        return {"workload": f"recent-window gather B={self.batch} L={self.layers} Hkv={self.heads} D={self.dim} "
                            f"page size {self.page_size}, context {self.context}, window {self.window}, bf16, "
                            f"random page permutation, {len(self.outs)} disjoint windows in rotation",
                "batch": self.batch}

    def cpu_baseline(self, threads):
        from oracle import kvwindow as okw
        torch.set_num_threads(threads)
        b, ctx = 1, 4096      # per-request work is the same; the pool is sized to what one request touches
        pages = ctx // self.page_size
        g = torch.Generator().manual_seed(5)
        table = torch.randperm(pages, generator=g).to(torch.int32)[None]
        k = torch.randn(self.layers, ctx, self.heads, self.dim, generator=g).to(torch.bfloat16)
        v = torch.randn(self.layers, ctx, self.heads, self.dim, generator=g).to(torch.bfloat16)
        seq = torch.tensor([ctx])
        med, n = time_cpu(lambda: okw.gather_window(k, v, table, seq, self.page_size, self.window))
        per_req = 2 * self.layers * 2 * self.heads * self.window * self.dim * 2
        return {"value": per_req * b / med / 1e9, "threads": threads,
                "sample": f"B={b} request, {self.layers} layers, context {ctx}, oracle torch-CPU gather, "
                          f"median of {n} runs"}


class SummaryUpdate:
    """Fused summary update (scores + merge, all layers in one launch), Qwen3-8B
    geometry: 36 layers, 32 query heads x 64 rows (256 rows per KV head), 8 KV
    heads, head_dim 128, 16 new rows per request (all accepted), batch 8."""

    copies, rotate = 2, ("state", "lse")

    name = "summary_update"
    dtype = "f32"
    metric = "summary update GB/s (algorithmic bytes) at 36L, 256 rows per KV head, W 16, B 8"
    unit = "GB/s"

    def __init__(self, dev, batch=8, layers=36, q_heads=32, kv_heads=8, rows=64, dim=128, width=16):
        self.dev, self.batch, self.layers = dev, batch, layers
        self.q_heads, self.kv_heads, self.rows, self.dim, self.width = q_heads, kv_heads, rows, dim, width
        g = torch.Generator(device=dev).manual_seed(41)
        self.query = torch.randn(layers, q_heads, rows, dim, generator=g, device=dev).to(torch.bfloat16)
        n = batch * width
        self.kc = torch.randn(layers, n, kv_heads, dim, generator=g, device=dev).to(torch.bfloat16)
        self.vc = torch.randn(layers, n, kv_heads, dim, generator=g, device=dev).to(torch.bfloat16)
        self.locs = torch.arange(n, device=dev).view(batch, width)
        self.lens = torch.full((batch,), width, dtype=torch.int32, device=dev)
        self.state = torch.randn(batch, layers, q_heads, rows, dim, generator=g, device=dev)
        self.lse = torch.randn(batch, layers, q_heads, rows, generator=g, device=dev)
        self.slots = torch.arange(batch, dtype=torch.int32, device=dev)
        self.bytes = (2 * self.state.numel() * 4 + 2 * self.lse.numel() * 4 + 2 * self.kc.numel() * 2
                      + self.query.numel() * 2)
        self.kernel = "summary_kernel"
        self.units = self.bytes / 1e9

    def step(self):
        from longspark_amd import summary
        summary.summary_update(query=self.query, key_cache=self.kc, value_cache=self.vc,
                               accepted_cache_locs=self.locs, accept_lens=self.lens, state_output=self.state,
                               state_lse=self.lse, softmax_scale=self.dim ** -0.5, state_slots=self.slots)

    def config(self):
        return {"workload": f"summary update B={self.batch} L={self.layers} Hq={self.q_heads} x S={self.rows} "
                            f"Hkv={self.kv_heads} D={self.dim} W={self.width}, fp32 state, bf16 q/k/v",
                "batch": self.batch}

    def cpu_baseline(self, threads):
        from oracle import summary as osm
        torch.set_num_threads(threads)
        b, layers = 1, self.layers
        g = torch.Generator().manual_seed(6)
        q = torch.randn(layers, self.q_heads, self.rows, self.dim, generator=g).to(torch.bfloat16)
        k = torch.randn(layers, b, self.width, self.kv_heads, self.dim, generator=g).to(torch.bfloat16)
        v = torch.randn(layers, b, self.width, self.kv_heads, self.dim, generator=g).to(torch.bfloat16)
        st = torch.randn(b, layers, self.q_heads, self.rows, self.dim, generator=g)
        ls = torch.randn(b, layers, self.q_heads, self.rows, generator=g)
        lens = torch.full((b,), self.width, dtype=torch.int32)

        def run():
            for l in range(layers):
                sc = osm.position_scores(q[l][None].expand(b, -1, -1, -1), k[l], self.dim ** -0.5)
                osm.merge_accepted_positions(st[:, l], ls[:, l], sc, v[l], lens)
        med, n = time_cpu(run)
        per_req = self.bytes / self.batch
        return {"value": per_req * b / med / 1e9, "threads": threads,
                "sample": f"B={b} request, {layers} layers, oracle torch-CPU score + merge per layer, "
                          f"median of {n} runs"}


class SoftmaxTempWorkload:
    """SoftmaxTemp.execute: fp32 softmax(logits / T) of B x K rows of 151,936
    bf16 logits, batch 128 x block 16 (one temperature per request)."""

    name = "softmax_temp"
    metric = "temperature softmax GB/s (algorithmic bytes) at 128x16x151936, bf16 in, fp32 out"
    unit = "GB/s"
    dtype = "f32"

    def __init__(self, dev, batch=128, width=16, vocab=V):
        from longspark_amd import workloads
        self.batch, self.width, self.vocab = batch, width, vocab
        self.logits, _ = workloads.greedy_inputs(batch, width, vocab, seed=71, device=dev, gen_device=dev)
        self.temps = torch.linspace(0.5, 1.5, batch, device=dev)
        rows = batch * width
        self.bytes = rows * vocab * 2 + rows * vocab * 4   # read the logits once, write the probabilities once
        self.units = self.bytes / 1e9
        self.kernel = "softmax_temp_resident_kernel"

    def step(self):
        from longspark_amd import dense
        return dense.softmax_temp(logits=self.logits, temperatures=self.temps, rows_per_request=self.width)

    def config(self):
        return {"workload": f"SoftmaxTemp B={self.batch} K={self.width} V={self.vocab} bf16 -> fp32",
                "batch": self.batch, "block": self.width, "vocab": self.vocab}

    def cpu_baseline(self, threads):
        from oracle import verify as ov
        torch.set_num_threads(threads)
        rows = 32
        x = self.logits[:rows].cpu()
        t = self.temps[:rows // self.width].cpu()
        med, n = time_cpu(lambda: ov.softmax_temp(x, t, self.width))
        return {"value": rows * self.vocab * 6 / med / 1e9, "threads": threads,
                "sample": f"{rows} rows x {self.vocab}, oracle torch-CPU softmax, median of {n} runs"}


class TargetProbsWorkload:
    """build_dflash_verify_target_probs: dense fp32 top-k 50 / top-p 0.95
    distribution (T 0.7) of B x K rows of 151,936 bf16 logits, 128 x 16."""

    name = "target_probs"
    metric = "dense target distribution GB/s (algorithmic bytes) at 128x16x151936, top-k 50, top-p 0.95"
    unit = "GB/s"
    dtype = "f32"

    def __init__(self, dev, batch=128, width=16, vocab=V):
        from longspark_amd import workloads
        self.batch, self.width, self.vocab = batch, width, vocab
        self.logits, _ = workloads.greedy_inputs(batch, width, vocab, seed=72, device=dev, gen_device=dev)
        self.params = workloads.SamplingParams.uniform(batch, temperature=0.7, top_k=50, top_p=0.95, device=dev)
        rows = batch * width
        self.bytes = rows * vocab * 2 + rows * vocab * 4   # read the logits once, write the dense rows once
        self.units = self.bytes / 1e9
        self.kernel = "ls_target_probs (all kernels of the call)"

    def step(self):
        from longspark_amd import dense
        p = self.params
        return dense.target_probs(logits=self.logits, temperatures=p.temperatures, rows_per_request=self.width,
                                  top_ks=p.top_ks, top_ps=p.top_ps, max_top_k=50, scan_hint=1)

    def config(self):
        return {"workload": f"dense target probabilities B={self.batch} K={self.width} V={self.vocab} bf16 -> "
                            "fp32, T 0.7, top-k 50, top-p 0.95", "batch": self.batch, "block": self.width,
                "vocab": self.vocab}

    def cpu_baseline(self, threads):
        from oracle import verify as ov
        torch.set_num_threads(threads)
        rows = 32
        x = self.logits[:rows].cpu()
        p = self.params
        b = rows // self.width
        med, n = time_cpu(lambda: ov.target_probs(x, temperatures=p.temperatures[:b].cpu(),
                                                  top_ks=p.top_ks[:b].cpu(), top_ps=p.top_ps[:b].cpu(),
                                                  min_ps=p.min_ps[:b].cpu(), rows_per_request=self.width))
        return {"value": rows * self.vocab * 6 / med / 1e9, "threads": threads,
                "sample": f"{rows} rows x {self.vocab}, oracle torch-CPU target distribution, median of {n} runs"}


class HbmCopy:
    """Plain device copy of 1 GiB (torch copy_), the calibration kernel for the
    FETCH_SIZE / WRITE_SIZE counters: it reads and writes exactly 1 GiB."""

    name = "hbm_copy"
    metric = "device copy GB/s (read + write) of 1 GiB"
    unit = "GB/s"

    def __init__(self, dev, nbytes=1 << 30):
        self.src = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=dev).fill_(1.0)
        self.dst = torch.empty_like(self.src)
        self.bytes = 2 * nbytes
        self.units = self.bytes / 1e9
        self.kernel = "copy"

    def step(self):
        self.dst.copy_(self.src)

    def config(self):
        return {"workload": "torch copy_ of 1 GiB bf16 (counter calibration)", "bytes": self.bytes // 2}

    def cpu_baseline(self, threads):
        torch.set_num_threads(threads)
        a = torch.empty(1 << 26, dtype=torch.bfloat16).fill_(1.0)
        b = torch.empty_like(a)
        med, n = time_cpu(lambda: b.copy_(a))
        return {"value": 2 * a.numel() * 2 / med / 1e9, "threads": threads,
                "sample": f"128 MiB host copy, median of {n} runs"}


class HbmFill:
    """Device fill of 1 GiB (torch fill_): the write-only rate, beside the
    copy's mixed read/write rate, for kernels whose traffic is mostly writes
    (SoftmaxTemp writes 2 bytes of fp32 output for every byte of bf16 it reads)."""

    name = "hbm_fill"
    metric = "device fill GB/s (write) of 1 GiB"
    unit = "GB/s"

    def __init__(self, dev, nbytes=1 << 30):
        self.dst = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
        self.bytes = nbytes
        self.units = self.bytes / 1e9
        self.kernel = "fill"
        self.dtype = "f32"

    def step(self):
        self.dst.fill_(1.0)

    def config(self):
        return {"workload": "torch fill_ of 1 GiB fp32 (write-only rate)", "bytes": self.bytes}

    def cpu_baseline(self, threads):
        torch.set_num_threads(threads)
        a = torch.empty(1 << 25, dtype=torch.float32)
        med, n = time_cpu(lambda: a.fill_(1.0))
        return {"value": a.numel() * 4 / med / 1e9, "threads": threads,
                "sample": f"128 MiB host fill, median of {n} runs"}


class ChainSampling:
    """chain_speculative_sampling_triton on dense fp32 target [B, K, V] and
    draft [B, K-1, V] probabilities (softmax of N(0, 3^2) logits at T 0.8,
    drafted tokens drawn from q), batch 128 x block 16."""

    copies, rotate = 7, ("p", "q")

    name = "chain_sampling"
    metric = "dense-q chain sampling GB/s (algorithmic bytes) at 128x16x151936 fp32 probabilities"
    unit = "GB/s"
    dtype = "f32"

    def __init__(self, dev, batch=128, width=16, vocab=V):
        from longspark_amd import accept
        g = torch.Generator(device=dev).manual_seed(81)
        self.batch, self.width, self.vocab = batch, width, vocab
        x = 3.0 * torch.randn(batch, width, vocab, generator=g, device=dev)
        self.p = torch.softmax(x / 0.8, dim=-1)
        x[:, :width - 1] += torch.randn(batch, width - 1, vocab, generator=g, device=dev)
        self.q = torch.softmax(x[:, :width - 1] / 0.8, dim=-1)
        del x
        self.cand = torch.zeros(batch, width, dtype=torch.int64, device=dev)
        self.cand[:, 1:] = torch.multinomial(self.q.reshape(-1, vocab), 1, generator=g).view(batch, width - 1)
        self.u = torch.rand(batch, width - 1, generator=g, device=dev)
        self.uf = torch.rand(batch, generator=g, device=dev)
        (self.ridx, self.nxt, self.sib, self.predicts, self.aidx,
         self.anum) = accept.chain_verify_buffers(bs=batch, draft_token_num=width, device=dev)
        self.bytes = batch * vocab * 4 * 2   # until count_rejected: p and q rows for every request
        self.units = self.bytes / 1e9
        self.kernel = "chain_kernel"

    def step(self):
        from longspark_amd import accept
        accept.chain_speculative_sampling_triton(
            self.predicts, self.aidx, self.anum, self.cand, self.ridx, self.nxt, self.sib, self.u, self.uf,
            self.p, self.q, 1.0, 1.0, True)
        return self.anum

    def count_rejected(self, anum):
        """Algorithmic bytes: per request the drafted tokens' p and q up to the
        first rejection, the bonus row of p, and q's row after a rejection."""
        n = anum.long().cpu()
        rejected = int((n < self.width - 1).sum())
        gathered = int((torch.clamp(n + 1, max=self.width - 1)).sum()) * 8
        self.bytes = self.batch * self.vocab * 4 + rejected * self.vocab * 4 + gathered
        self.units = self.bytes / 1e9
        self.rejected = rejected

    def config(self):
        return {"workload": f"chain sampling B={self.batch} K={self.width} V={self.vocab} fp32 p and q",
                "batch": self.batch, "block": self.width, "vocab": self.vocab,
                "rejected_requests": getattr(self, "rejected", None)}

    def cpu_baseline(self, threads):
        from oracle import verify as ov
        torch.set_num_threads(threads)
        b = 8
        p, q = self.p[:b].cpu(), self.q[:b].cpu()
        cand, u, uf = self.cand[:b].cpu(), self.u[:b].cpu(), self.uf[:b].cpu()
        med, n = time_cpu(lambda: ov.chain_speculative_sampling(candidates=cand, uniform_samples=u, uniform_final=uf,
                                                                 target_probs_3d=p, draft_probs_3d=q))
        return {"value": b * self.vocab * 8 / med / 1e9, "threads": threads,
                "sample": f"{b} requests, oracle torch-CPU chain sampling, median of {n} runs"}


class SampleStep:
    """sample_step_tokens_with_q: the drafter's per-step exponential race with
    the sampled q over fp32 logits [128, 151,936] and fp32 Exp(1) noise of the
    same shape (one proposal step of a batch of 128)."""

    copies, rotate = 7, ("logits", "noise")

    name = "sample_step"
    metric = "proposal-step sampling GB/s (algorithmic bytes) at 128x151936 fp32 logits + fp32 noise"
    unit = "GB/s"
    dtype = "f32"

    def __init__(self, dev, batch=128, vocab=V):
        g = torch.Generator(device=dev).manual_seed(84)
        self.batch, self.vocab = batch, vocab
        self.logits = 3.0 * torch.randn(batch, vocab, generator=g, device=dev)
        self.temps = torch.linspace(0.5, 1.5, batch, device=dev)
        self.noise = torch.empty(batch, vocab, device=dev).exponential_(1, generator=g)
        self.bytes = batch * vocab * 8     # every logit and noise value read once
        self.units = self.bytes / 1e9
        self.kernel = "sample_step_kernel"

    def step(self):
        from longspark_amd import sample
        return sample.sample_step_tokens_with_q(step_logits=self.logits, temperatures=self.temps,
                                                exp_noise=self.noise)

    def config(self):
        return {"workload": f"proposal step B={self.batch} V={self.vocab} fp32 logits + fp32 noise",
                "batch": self.batch, "vocab": self.vocab}

    def cpu_baseline(self, threads):
        from oracle import verify as ov
        torch.set_num_threads(threads)
        b = 16
        x, t, n = self.logits[:b].cpu(), self.temps[:b].cpu(), self.noise[:b].cpu()
        med, k = time_cpu(lambda: ov.sample_step_tokens_with_q(x, t, n))
        return {"value": b * self.vocab * 8 / med / 1e9, "threads": threads,
                "sample": f"{b} rows, oracle torch-CPU exponential race, median of {k} runs"}


class Global16Prefill:
    """Prefill summary initialisation (run_prefill_global_attention of every
    selected layer) at Qwen3-14B geometry: 5 selected layers, 40 query and 8
    KV heads, 16 summary slots, head_dim 128, one request with a 131,072-token
    prefix in bf16 pools of page size 1, the prefix's locations a random
    permutation of 16-token pages.  All five layers go in one launch (plus the
    split combine)."""

    name = "global16_prefill"
    metric = "prefill summary initialisation GB/s (algorithmic bytes) at 5L x 8 Hkv x D128, prefix 131072, B 1"
    unit = "GB/s"
    dtype = "bf16"

    def __init__(self, dev, batch=1, layers=5, q_heads=40, kv_heads=8, rows=16, dim=128, prefix=131072, page=16):
        self.batch, self.layers, self.q_heads, self.kv_heads = batch, layers, q_heads, kv_heads
        self.rows, self.dim, self.prefix = rows, dim, prefix
        g = torch.Generator(device=dev).manual_seed(57)
        n = batch * prefix
        pages = torch.randperm(n // page, generator=g, device=dev).view(batch, prefix // page)
        self.table = (pages[:, :, None] * page + torch.arange(page, device=dev)).view(batch, prefix).to(torch.int32)
        self.lens = torch.full((batch,), prefix, dtype=torch.int32, device=dev)
        self.k = [torch.randn(n, kv_heads, dim, generator=g, device=dev).to(torch.bfloat16) for _ in range(layers)]
        self.v = [torch.randn(n, kv_heads, dim, generator=g, device=dev).to(torch.bfloat16) for _ in range(layers)]
        self.query = torch.randn(layers, q_heads, rows, dim, generator=g, device=dev).to(torch.bfloat16)
        self.out = torch.empty(batch, layers, q_heads, rows, dim, device=dev)
        self.lse = torch.empty(batch, layers, q_heads, rows, device=dev)
        kv = 2 * layers * batch * prefix * kv_heads * dim * 2
        self.bytes = kv + self.query.numel() * 2 + self.out.numel() * 4 + self.lse.numel() * 4 + batch * prefix * 4
        self.units = self.bytes / 1e9
        self.kernel = "prefill_kernel + prefill_combine_kernel"

    def step(self):
        from longspark_amd import summary
        return summary.prefill_global_attention(query=self.query, key_cache=self.k, value_cache=self.v,
                                                page_table=self.table, cache_seqlens=self.lens,
                                                softmax_scale=self.dim ** -0.5, output=self.out, lse=self.lse)

    def config(self):
        return {"workload": f"Global16 prefill B={self.batch} L={self.layers} Hq={self.q_heads} x S={self.rows} "
                            f"Hkv={self.kv_heads} D={self.dim} prefix {self.prefix}, bf16 K/V, page size 1 "
                            "(16-token pages permuted)", "batch": self.batch}

    def cpu_baseline(self, threads):
        from oracle import summary as osm
        torch.set_num_threads(threads)
        n = 8192             # per-token work is the same at every prefix length
        g = torch.Generator().manual_seed(8)
        q = torch.randn(self.q_heads, self.rows, self.dim, generator=g).to(torch.bfloat16)
        k = torch.randn(n, self.kv_heads, self.dim, generator=g).to(torch.bfloat16)
        v = torch.randn(n, self.kv_heads, self.dim, generator=g).to(torch.bfloat16)
        table = torch.randperm(n, generator=g)[None].to(torch.int32)
        lens = torch.tensor([n], dtype=torch.int32)
        med, reps = time_cpu(lambda: osm.prefill_global_attention(q, k, v, table, lens, self.dim ** -0.5,
                                                                   dtype=torch.float32))
        per_layer = 2 * n * self.kv_heads * self.dim * 2
        return {"value": per_layer / med / 1e9, "threads": threads,
                "sample": f"one layer, prefix {n}, oracle torch-CPU fp32 attention, median of {reps} runs"}


class DraftAttention:
    """fused_global_local_raw_attention: one drafter attention step over the
    three views for a batch of 128 requests, 32 query and 8 KV heads,
    head_dim 128, 7 query rows; every request's Raw256 window full (256 rows,
    page size 1, rows scattered over a pool of 128 x 256 slots), 16 summary
    rows per query head from the fp32 state, 7 local rows under a causal
    in-block mask."""

    copies, rotate = 5, ("q", "gk", "gv", "lk", "lv", "mask", "kc", "vc", "pt", "out")

    name = "draft_attention"
    metric = "drafter attention GB/s (algorithmic bytes) at B=128, 32 Hq / 8 Hkv, D 128, Raw256 + Global16 + Local7"
    unit = "GB/s"
    dtype = "bf16"

    def __init__(self, dev, batch=128, q_heads=32, kv_heads=8):
        g = torch.Generator(device=dev).manual_seed(63)
        self.batch, self.q_heads, self.kv_heads = batch, q_heads, kv_heads
        bf = torch.bfloat16
        self.q = (0.3 * torch.randn(batch, q_heads, 7, 128, generator=g, device=dev)).to(bf)
        self.gk = (0.3 * torch.randn(batch, q_heads, 16, 128, generator=g, device=dev)).to(bf)
        self.gv = torch.randn(batch, q_heads, 16, 128, generator=g, device=dev)
        self.slots = torch.arange(batch, dtype=torch.int32, device=dev)
        self.lk = (0.3 * torch.randn(batch, kv_heads, 7, 128, generator=g, device=dev)).to(bf)
        self.lv = torch.randn(batch, kv_heads, 7, 128, generator=g, device=dev).to(bf)
        self.mask = torch.ones(7, 7, dtype=torch.bool, device=dev).tril().expand(batch, 7, 7).contiguous()
        pool = batch * 256
        self.kc = (0.3 * torch.randn(pool, 1, kv_heads, 128, generator=g, device=dev)).to(bf)
        self.vc = torch.randn(pool, 1, kv_heads, 128, generator=g, device=dev).to(bf)
        self.pt = torch.randperm(pool, generator=g, device=dev).to(torch.int32).view(batch, 256)
        self.rl = torch.full((batch,), 256, dtype=torch.int32, device=dev)
        self.out = torch.empty_like(self.q)
        raw = 2 * batch * kv_heads * 256 * 128 * 2
        per_head = 16 * 128 * 2 + 16 * 128 * 4 + 2 * 7 * 128 * 2      # summary keys, fp32 state, query + output
        self.bytes = raw + batch * q_heads * per_head + 2 * self.lk.numel() * 2 + self.pt.numel() * 4 \
            + self.mask.numel()
        self.units = self.bytes / 1e9
        self.kernel = "draft_attention_kernel"

    def step(self):
        from longspark_amd import draft_attention
        return draft_attention.fused_global_local_raw_attention(
            query=self.q, global_keys=self.gk, global_values=self.gv, state_slots=self.slots, local_keys=self.lk,
            local_values=self.lv, local_attention_mask=self.mask, key_cache=self.kc, value_cache=self.vc,
            page_table=self.pt, raw_lengths=self.rl, output=self.out, softmax_scale=128 ** -0.5)

    def config(self):
        return {"workload": f"drafter attention B={self.batch} Hq={self.q_heads} Hkv={self.kv_heads} D=128, "
                            "7 rows over Raw256 (full) + Global16 + Local7", "batch": self.batch}

    def cpu_baseline(self, threads):
        from oracle import draft_attention as oda
        torch.set_num_threads(threads)
        b = 2
        args = [t[:b].cpu() for t in (self.q, self.gk, self.gv)] + [torch.arange(b, dtype=torch.int32)] + \
               [t[:b].cpu() for t in (self.lk, self.lv, self.mask)] + [self.kc.cpu(), self.vc.cpu()] + \
               [t[:b].cpu() for t in (self.pt, self.rl)]
        med, n = time_cpu(lambda: oda.fused_global_local_raw_attention(*args, 128 ** -0.5))
        return {"value": self.bytes * b / self.batch / med / 1e9, "threads": threads,
                "sample": f"{b} requests, oracle torch-CPU per (request, query head), median of {n} runs"}


class DraftMerge(DraftAttention):
    """fused_global_local_raw_merge: the merge step after a separate window
    attention, for the same batch and heads as the one-kernel workload: the
    window attention's bf16 output [B*7, Hq, 128] and fp32 LSE [B*7, Hq]
    merged with the 16 summary rows (fp32 state) and 7 local rows per query
    head."""

    copies, rotate = 13, ("q", "gk", "gv", "lk", "lv", "mask", "raw_out", "raw_lse", "out")

    name = "draft_merge"
    metric = "drafter merge GB/s (algorithmic bytes) at B=128, 32 Hq / 8 Hkv, D 128, window output + Global16 + Local7"

    def __init__(self, dev, batch=128, q_heads=32, kv_heads=8):
        super().__init__(dev, batch=batch, q_heads=q_heads, kv_heads=kv_heads)
        g = torch.Generator(device=dev).manual_seed(64)
        self.kc = self.vc = self.pt = None
        self.raw_out = torch.randn(batch * 7, q_heads, 128, generator=g, device=dev).to(torch.bfloat16)
        self.raw_lse = 2.0 * torch.randn(batch * 7, q_heads, generator=g, device=dev)
        # per query head: query, window output and merged output rows (bf16), window LSE, summary keys (bf16)
        # and fp32 state; per KV head the local K and V rows; the local mask
        per_head = 3 * 7 * 128 * 2 + 7 * 4 + 16 * 128 * 2 + 16 * 128 * 4
        self.bytes = batch * q_heads * per_head + 2 * self.lk.numel() * 2 + self.mask.numel()
        self.units = self.bytes / 1e9
        self.kernel = "draft_merge_kernel"

    def step(self):
        from longspark_amd import draft_attention
        return draft_attention.fused_global_local_raw_merge(
            query=self.q, global_keys=self.gk, global_values=self.gv, state_slots=self.slots, local_keys=self.lk,
            local_values=self.lv, local_attention_mask=self.mask, raw_output=self.raw_out, raw_lse=self.raw_lse,
            output=self.out, softmax_scale=128 ** -0.5)

    def config(self):
        return {"workload": f"drafter merge B={self.batch} Hq={self.q_heads} Hkv={self.kv_heads} D=128, "
                            "window output + LSE merged with Global16 + Local7", "batch": self.batch}

    def cpu_baseline(self, threads):
        from oracle import draft_attention as oda
        torch.set_num_threads(threads)
        b = 8
        args = [t[:b].cpu() for t in (self.q, self.gk, self.gv)] + [torch.arange(b, dtype=torch.int32)] + \
               [t[:b].cpu() for t in (self.lk, self.lv, self.mask)] + \
               [self.raw_out[:7 * b].cpu(), self.raw_lse[:7 * b].cpu()]
        med, n = time_cpu(lambda: oda.fused_global_local_raw_merge(*args, 128 ** -0.5))
        return {"value": self.bytes * b / self.batch / med / 1e9, "threads": threads,
                "sample": f"{b} requests, oracle torch-CPU merge, median of {n} runs"}


class FullRound:
    """One verify-and-refresh round at Qwen3-14B geometry: 40 layers, 40 query
    and 8 KV heads, head_dim 128, vocab 151,936, batch 128, block 16, contexts
    U[8K, 32K] in a paged bf16 cache (page 16).  A round runs the penalty
    tables and the fused stochastic verify (T 0.7, top-k 50, top-p 0.95,
    repetition 1.05 over a 2048-token Zipf history), the 256-token window
    gather of every layer, and the summary update (52 rows per query head,
    260 per KV head) with each request's committed rows (accepted drafts plus
    the bonus) read from the cache.  The cache pool holds the pages the
    windows touch plus as many distractor pages; page-table entries outside
    the windows alias random pool pages (the values are random, so the access
    pattern is kept), since 128 contexts of this size do not fit in HBM."""

    name = "full_round"
    metric = "per-round GB/s (algorithmic bytes): verify + window gather + summary update, Qwen3-14B, B=128"
    unit = "GB/s"
    dtype = "bf16"

    def __init__(self, dev, batch=128, width=16, layers=40, q_heads=40, kv_heads=8, dim=128, rows=52, page=16,
                 window=256):
        self.verify = StochasticVerify(dev, batch=batch, width=width)
        self.batch, self.width, self.layers, self.dim, self.window, self.page = batch, width, layers, dim, window, page
        self.q_heads, self.kv_heads, self.rows = q_heads, kv_heads, rows
        from longspark_amd import workloads
        r = workloads.full_round_refresh_inputs(dev, batch=batch, width=width, layers=layers, q_heads=q_heads,
                                                kv_heads=kv_heads, dim=dim, rows=rows, page=page, window=window)
        self.table, self.seq, self.k, self.v, self.locs = r["table"], r["seq"], r["k"], r["v"], r["locs"]
        self.query, self.state, self.lse = r["query"], r["state"], r["lse"]
        self.out = torch.empty(batch, layers, 2, kv_heads, window, dim, dtype=torch.bfloat16, device=dev)
        self.committed = width * batch
        self._set_bytes(self.verify.rows * V * 2 + batch * V * 4)
        self.kernel = "full round (all kernels of the round)"

    def _set_bytes(self, verify_bytes):
        gather = 2 * self.out.numel() * 2
        summary = (2 * self.state.numel() * 4 + 2 * self.lse.numel() * 4 + self.query.numel() * 2
                   + self.committed * self.layers * 2 * self.kv_heads * self.dim * 2)
        self.parts = {"verify": verify_bytes, "window_gather": gather, "summary_update": summary}
        self.bytes = sum(self.parts.values())
        self.units = self.bytes / 1e9

    def step(self):
        from longspark_amd import kvwindow, summary
        acc, _ = self.verify.step()
        kvwindow.gather_window(self.k, self.v, self.table, self.seq, page_size=self.page, window=self.window,
                               out=self.out)
        lens = (acc + 1).clamp_(0, self.width)   # committed rows: accepted drafts + the bonus
        summary.summary_update(query=self.query, key_cache=self.k, value_cache=self.v, accepted_cache_locs=self.locs,
                               accept_lens=lens, state_output=self.state, state_lse=self.lse,
                               softmax_scale=self.dim ** -0.5)
        return acc, lens

    def count_rejected(self, out):
        acc, lens = out
        self.verify.count_rejected((acc, None))
        self.committed = int(lens.sum().item())
        self._set_bytes(self.verify.kernel_bytes + self.batch * self.verify.cfg["history_len"] * 4)

    def config(self):
        return {"workload": f"full round, Qwen3-14B geometry: verify B={self.batch} K={self.width} V={V} bf16 "
                            f"(T 0.7, top-k 50, top-p 0.95, repetition 1.05, 2048-token history) + window gather "
                            f"{self.window} x {self.layers} layers x {self.kv_heads} KV heads x D {self.dim} "
                            f"(contexts U[8K, 32K], page {self.page}) + summary update "
                            f"{self.q_heads}x{self.rows} rows per layer over the committed rows",
                "batch": self.batch, "block": self.width, "vocab": V, "layers": self.layers,
                "committed_rows": self.committed,
                "bytes_per_part": self.parts}

    def cpu_baseline(self, threads):
        from oracle import kvwindow as okw
        from oracle import summary as osm
        verify = self.verify.cpu_baseline(threads)       # B=2 requests
        t_verify = 2 * self.width / verify["rows_per_s"]
        g = torch.Generator().manual_seed(9)
        ctx = 4096
        table = torch.randperm(ctx // self.page, generator=g).to(torch.int32)[None]
        k = torch.randn(self.layers, ctx, self.kv_heads, self.dim, generator=g).to(torch.bfloat16)
        v = torch.randn(self.layers, ctx, self.kv_heads, self.dim, generator=g).to(torch.bfloat16)
        t_gather, _ = time_cpu(lambda: okw.gather_window(k, v, table, torch.tensor([ctx]), self.page, self.window))
        q = torch.randn(self.layers, self.q_heads, self.rows, self.dim, generator=g).to(torch.bfloat16)
        kn = torch.randn(self.layers, 1, self.width, self.kv_heads, self.dim, generator=g).to(torch.bfloat16)
        st = torch.randn(1, self.layers, self.q_heads, self.rows, self.dim, generator=g)
        ls = torch.randn(1, self.layers, self.q_heads, self.rows, generator=g)
        lens = torch.full((1,), self.width, dtype=torch.int32)

        def run():
            for layer in range(self.layers):
                sc = osm.position_scores(q[layer][None], kn[layer], self.dim ** -0.5)
                osm.merge_accepted_positions(st[:, layer], ls[:, layer], sc, kn[layer], lens)
        t_summary, n = time_cpu(run)
        per_request = self.bytes / self.batch
        t = t_verify / 2 + t_gather + t_summary
        return {"value": per_request / t / 1e9, "threads": threads,
                "sample": f"one request's round: oracle verify (timed at B=2), gather ({self.layers} layers, "
                          f"context {ctx}) and summary update ({self.layers} layers), torch-CPU, median of {n} runs"}


class _BatchInfo(SimpleNamespace):
    """The sampling-info fields the verify logit adjustments read (one entry per request)."""

    def __len__(self):
        return self.temperatures.shape[0]


class AdjustLogits:
    """apply_dflash_verify_logits_adjustments (overlap path): fp32
    acc_linear_penalties and logit_bias [B, V] added in bf16 to every row of
    each request, in place on [B*K, V] bf16 logits, batch 128 x block 16."""

    copies, rotate = 2, ("logits",)

    name = "adjust_logits"
    metric = "verify logit adjustments GB/s (algorithmic bytes) at 128x16x151936 bf16"
    unit = "GB/s"
    dtype = "bf16"

    def __init__(self, dev, batch=128, width=16, vocab=V):
        from longspark_amd import workloads
        self.batch, self.width, self.vocab = batch, width, vocab
        self.logits, _ = workloads.greedy_inputs(batch, width, vocab, seed=82, device=dev, gen_device=dev)
        g = torch.Generator(device=dev).manual_seed(83)
        acc = -0.05 * torch.randint(0, 3, (batch, vocab), generator=g, device=dev).float()
        lb = torch.zeros(batch, vocab, device=dev)
        lb[:, ::101] = 0.01
        self.info = _BatchInfo(acc_linear_penalties=acc, logit_bias=lb, penalizer_orchestrator=None,
                               vocab_mask=None, has_custom_logit_processor=False,
                               temperatures=torch.ones(batch, 1, device=dev))
        rows = batch * width
        self.bytes = rows * vocab * 2 * 2 + 2 * batch * vocab * 4   # logits read + written, two fp32 [B, V]
        self.units = self.bytes / 1e9
        self.kernel = "request_bias_kernel"

    def step(self):
        from longspark_amd import penalties
        penalties.apply_dflash_verify_logits_adjustments(next_token_logits=self.logits, sampling_info=self.info,
                                                         draft_token_num=self.width)

    def config(self):
        return {"workload": f"verify logit adjustments B={self.batch} K={self.width} V={self.vocab} bf16",
                "batch": self.batch, "block": self.width, "vocab": self.vocab}

    def cpu_baseline(self, threads):
        torch.set_num_threads(threads)
        b = 4
        x = self.logits[:b * self.width].cpu().view(b, self.width, self.vocab)
        acc = self.info.acc_linear_penalties[:b].cpu()
        lb = self.info.logit_bias[:b].cpu()

        def run():  # the reference's tensor operations (dflash_utils.py:193-213) on the CPU
            x.add_(acc.to(x.dtype)[:, None, :])
            x.add_(lb.to(x.dtype)[:, None, :])
        med, n = time_cpu(run)
        return {"value": (b * self.width * self.vocab * 4 + 2 * b * self.vocab * 4) / med / 1e9,
                "threads": threads, "sample": f"{b} requests, torch-CPU adds of the reference, median of {n} runs"}


WORKLOADS = {w.name: w for w in (GreedyVerify, StochasticVerify, StochasticVerifyHighAccept, WindowGather, SummaryUpdate, SoftmaxTempWorkload,
                                  TargetProbsWorkload, ChainSampling, AdjustLogits, SampleStep, Global16Prefill, DraftAttention,
                                  DraftMerge, FullRound, HbmCopy, HbmFill)}
DEFAULT_WORKLOAD = "verify_sample"


def _clone(x):
    if torch.is_tensor(x):
        return x.clone()
    if isinstance(x, dict):
        return {k: _clone(v) for k, v in x.items()}
    if isinstance(x, list):
        return [_clone(v) for v in x]
    return x


class Rotation:
    """Input rotation: a workload whose tensors fit in the 256 MB last-level
    cache (or come close) names them in ``rotate``; ``copies`` - 1 clones go
    to distinct memory and consecutive steps use the copies in turn, so one
    cycle touches at least about 1 GB and no step re-reads lines an earlier
    step left in the cache.  The copies hold equal values, so every step
    computes the same result."""

    def __init__(self, wl):
        self.wl = wl
        names = getattr(wl, "rotate", ())
        n = getattr(wl, "copies", 1) if names else 1
        self.sets = [{k: getattr(wl, k) for k in names}]
        self.sets += [{k: _clone(getattr(wl, k)) for k in names} for _ in range(n - 1)]
        self.turn = 0

    def step(self):
        if len(self.sets) > 1:
            for k, v in self.sets[self.turn % len(self.sets)].items():
                setattr(self.wl, k, v)
            self.turn += 1
        return self.wl.step()


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the hot path is per-GPU; "
              "multi-GPU sharding is a design note, not a measured configuration)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 2

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    wl = WORKLOADS[args.workload](dev)
    stream = torch.cuda.current_stream(dev)
    rot = Rotation(wl)

    out = None
    for _ in range(args.warmup):
        out = rot.step()
    torch.cuda.synchronize()
    if hasattr(wl, "count_rejected"):
        wl.count_rejected(out if out is not None else rot.step())
    if hasattr(wl, "arm_timing"):
        wl.arm_timing(args.steps)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps):
        rot.step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall / args.steps * 1e3
    step_gpu_ms = start.elapsed_time(end) / args.steps
    units = getattr(wl, "units", None)
    value = (units if units is not None else wl.rows) / (ms_per_step / 1e3)
    kernels = wl.kernel_times_ms() if hasattr(wl, "kernel_times_ms") else {wl.kernel: step_gpu_ms}
    kernel_ms = kernels[wl.kernel]
    kernel_bytes = getattr(wl, "kernel_bytes", wl.bytes)
    achieved = kernel_bytes / (kernel_ms / 1e3) / 1e9

    cpu = None
    if not args.no_cpu_baseline:
        ncores = len(os.sched_getaffinity(0))
        allc = wl.cpu_baseline(ncores)
        four = wl.cpu_baseline(4)
        key = "rows_per_s" if "rows_per_s" in allc else "value"
        cpu = {"value": allc[key], "unit": getattr(wl, "unit", "rows/s"), "cores": ncores, "kind": "port",
               "sample": allc["sample"], "cpu_model": _cpu_model(),
               "value_4_threads": four[key]}

    line = {
        "metric": getattr(wl, "metric", "verified rows/sec at Bx16x151936 bf16"),
        "value": value,
        "unit": getattr(wl, "unit", "rows/s"),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": getattr(wl, "dtype", "bf16"),
        "data": "synthetic",
        "config": {**wl.config(), "input_copies": len(rot.sets)},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": TRAFFIC.get(wl.kernel, (None,))[0],
                     "traffic_source": TRAFFIC.get(wl.kernel, (None, None))[1], "kernel": wl.kernel,
                     "kernel_avg_us": kernel_ms * 1e3, "algorithmic_bytes": kernel_bytes},
        "step": {"gpu_us": step_gpu_ms * 1e3, "algorithmic_bytes": wl.bytes,
                 "gbs": wl.bytes / (step_gpu_ms / 1e3) / 1e9,
                 "kernels_us": {k: v * 1e3 for k, v in kernels.items()}},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
