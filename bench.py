#!/usr/bin/env python3
"""bench.py -- the headline benchmark: BASELINE config 4 on one MI355X.

Workload (config 4): a Qwen3-8B-shaped decoder (36 layers, hidden 4096,
32 q / 8 kv heads, head_dim 128, MLP 12288, vocab 151936) with random-init
int4 weights (the BASELINE pack: symmetric, group 32 along K, f16 scales; the
embedding int8), continuous batching through the library's Scheduler
(scheduler.go semantics, chunk 512): 128 decoding sequences whose contexts are
lognormal(median 1024, sigma 1.0) clipped to [16, 8192] tokens, plus 2 prefill
chunks of 512 tokens per step, page size 16, f16 KV pool, greedy sampling on
the device. Arrivals and completions are seeded: each request has a prompt of
the same lognormal length and an output budget U[100, 300]; a finished
sequence frees its slot and the next arrival is admitted when fewer than two
requests are mid-prefill. The initial 128 decoders are admitted with their
context already in the pool (synthetic KV), so step 1 is already steady state.

A step is one Scheduler.Step: one batched forward pass over ~1152 rows. By
default the scheduler runs in overlap mode: the host schedules and submits
step k+1 while the device runs step k (the decode rows take their tokens from
the device argmax), which runs the same steps and produces the same tokens as
the synchronous mode (--sync).
value = output tokens (sampleable tokens produced) / wall time of the timed
steps, inputs resident in HBM. The roofline object is the ragged paged
attention kernel (the metric's "paged-attn HBM GB/s"): algorithmic bytes per
launch (every cached position a claimed row reads, K+V of the 8 kv heads
once = 4096 B per position, plus 16 KiB per query row for q in and out, both
f16)
divided by its duration, bracketed with HIP events on the launch stream over
the timed steps (the launches of every 4th layer: each layer's attention does
the same work, and each event record leaves the device idle a few us).
cpu_baseline times tgo's CPU path restated (oracle/) on one of the timed
steps: the step with 1 and with 2 layers, extrapolated to 36.
"""
import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

C4 = dict(layers=36, hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=12288, vocab=151936,
          rms_eps=1e-6, rope_theta=1e6, block=16)
SEED = 2026
POOL = 400_000          # positions in the shared KV pool (59 GB of f16 K+V)
SLOTS = 136             # 128 decoders + 2 prefilling + headroom
CHUNK = 512
DECODERS = 128
PREFILLING = 2
# BASELINE config 5 (bench.py --config c5, a second workload; the default is config 4)
C5 = dict(layers=64, hidden=5120, heads=64, kv_heads=8, head_dim=128, ffn=25600, vocab=151936,
          rms_eps=1e-6, rope_theta=1e6, block=16)
C5_PREFIX = 2048        # tokens every sequence begins with (128 shared pages)
# BASELINE config 1 (bench.py --config c1): Qwen3-0.6B-shaped, f16 weights, one step
C1 = dict(layers=28, hidden=1024, heads=16, kv_heads=8, head_dim=128, ffn=3072, vocab=151936,
          rms_eps=1e-6, rope_theta=1e6, block=16)
C1_CONTEXTS = (37, 300, 511)  # the decoding sequences' contexts
C1_CHUNK = 64                 # the fresh sequence's prefill chunk
C1_POOL = 4096
C5_DECODERS = 256
C5_CHUNK = 1024
C5_POOL = 330_000       # positions (86 GB of f16 K+V at 64 layers)
HBM_PEAK = 8000.0       # GB/s, MI355X published
PROFILE_STRIDE = 4      # attention launches timed: those of every 4th layer
PROFILE_STEPS = 3       # steps with every kernel kind timed, after each timed phase
MFMA_F16_PEAK = 2500.0  # TFLOP/s dense f16, MI355X published


def lognormal_len(rng):
    return int(min(8192, max(16, round(math.exp(math.log(1024) + 1.0 * rng.standard_normal())))))


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None,
                   help="timed steps (default 200; 10 with --config c5, whose pool of 330k "
                        "positions holds about 20 steps of its arrivals and growth)")
    p.add_argument("--warmup", type=int, default=None, help="untimed steps (default 10; 3 for c5)")
    p.add_argument("--precision", type=int, default=1,
                   help="1 (default): tgo's f32 arithmetic (activations and probabilities as "
                        "f16 hi+lo, the exact dequantized weights as f16 hi+lo; within 2e-3 of "
                        "tgo's CPU path through all 36 layers); 0: f16 operands (faster, "
                        "~5e-3 after 36 layers)")
    p.add_argument("--fast-steps", type=int, default=40,
                   help="after the headline, this many mixed and decode-only steps with f16 "
                        "operands (precision 0) for the line's fast_path object (0: skip)")
    p.add_argument("--form", type=int, default=3, help="weight form (3: int4 sym g32-K, 2: tgo int4)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--sync", action="store_true",
                   help="synchronous steps (tgo's Batch.step: pack, submit, wait, read back); "
                        "the default overlaps the host's scheduling of step k+1 with the "
                        "device's step k (the same steps and tokens)")
    p.add_argument("--config", default="c4", choices=["c4", "c5", "c1"],
                   help="c4 (default): the headline workload; c5: BASELINE config 5, Qwen3-32B "
                        "int8 with a 2048-token prefix shared by 256 sequences (prefix-shared "
                        "attention on); c1: BASELINE config 1, Qwen3-0.6B f16, its one step "
                        "(3 decodes + a 64-token chunk) replayed, tgo's CPU path timed beside it")
    p.add_argument("--cascade", type=int, default=2,
                   help="config 5: group decode rows whose page tables share a prefix when at "
                        "least this many do (0: off, every sequence reads its own prefix)")
    p.add_argument("--phase", default="both", choices=["both", "mixed", "decode"],
                   help="profiling runs: mixed steps only, or straight to the decode-only steps "
                        "(the default line runs both)")
    p.add_argument("--decode-steps", type=int, default=100,
                   help="after the headline steps, this many decode-only steps (the 128 decoders "
                        "with no prefill chunk) for the decode-dominated figures (0: skip)")
    p.add_argument("--copy-probe-mib", type=int, default=0,
                   help="before the workload, run one plain f32 copy kernel (torch.neg) over this "
                        "many MiB: the known-size dispatch that scales the HBM byte counters")
    args = p.parse_args()
    if args.steps is None:
        args.steps = {"c5": 10, "c1": 500}.get(args.config, 200)
    if args.warmup is None:
        args.warmup = {"c5": 3, "c1": 20}.get(args.config, 10)
    return args


def copy_probe(mib):
    """One elementwise kernel that reads and writes exactly mib MiB each (y = -x, f32)."""
    import torch
    x = torch.ones(mib << 18, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    torch.neg(x, out=y)
    torch.cuda.synchronize()
    print("copy probe: %d MiB read + %d MiB written by one torch.neg dispatch" % (mib, mib),
          file=sys.stderr, flush=True)
    del x, y
    torch.cuda.empty_cache()


def achievable_peaks(ctx):
    """What this box reaches, measured before the timed work, beside the published peaks:
    the library's streaming read of 2 GiB and its dense f16 MFMA loop (tgohip_probe_peaks,
    medians of 5 timed launches)."""
    read_gbps, mfma_tflops = ctx.probe_peaks(2 << 30, 5)
    return {
        "read_gbps": round(read_gbps, 1),
        "mfma_f16_tflops": round(mfma_tflops, 1),
        "how": "tgohip_probe_peaks before the timed region: a grid-stride read of 2 GiB "
               "(16-byte non-temporal loads) and independent v_mfma_f32_32x32x16_f16 chains on every CU; "
               "medians of 5",
    }


class Workload:
    """Seeded arrivals and completions driving the library's Scheduler so that
    every step carries 128 decodes and 2 prefill chunks of 512.

    Arrival prompts are lognormal(median 1024, sigma 1) clipped to [16, 8192]
    and rounded up to whole chunks, so each chunk is exactly 512 tokens. When a
    request finishes its prompt it starts decoding, and the decoder closest to
    its output budget (U[100,300], seeded) completes, freeing its slot for the
    next arrival: 128 decoders and 2 prefilling requests at every step."""

    def __init__(self, tgo, ctx, seed):
        self.rng = np.random.default_rng(seed)
        self.sched = tgo.Scheduler(ctx, SLOTS, chunk=CHUNK, reserve=512,
                                   max_rows=PREFILLING * CHUNK + DECODERS)
        self.target = {}
        self.made = {}
        self.decoding = set()
        self.V = C4["vocab"]
        used = 0
        for _ in range(DECODERS):
            L = lognormal_len(self.rng)
            out = int(self.rng.integers(100, 301))
            prompt = [int(t) for t in self.rng.integers(0, self.V, L)]
            slot = self.sched.admit_prefilled(prompt, int(self.rng.integers(0, self.V)),
                                              reserve=out)
            # already part-way through its answer: completions are spread from step 1
            self.target[slot], self.made[slot] = out, int(self.rng.integers(0, out))
            self.decoding.add(slot)
            used += L + out
        self.used_positions = used
        self.contexts = [self.sched.length(s) for s in sorted(self.decoding)]
        self.admit_arrivals()

    def admit_arrivals(self):
        while self.sched.prefilling() < PREFILLING:
            L = CHUNK * ((lognormal_len(self.rng) + CHUNK - 1) // CHUNK)
            out = int(self.rng.integers(100, 301))
            prompt = [int(t) for t in self.rng.integers(0, self.V, L)]
            slot = self.sched.admit(prompt, reserve=out)
            self.target[slot], self.made[slot] = out, 0

    def decide(self, produced, tokens=None):
        """The books after a step: produced is [(slot, done)]. Each request that started
        decoding retires the decoder nearest its budget; arrivals refill the prefill
        slots. tokens ({slot: token}, synchronous mode) are fed back; in overlap mode the
        scheduler feeds them on the device. The decisions need no token values, so in
        overlap mode they are taken before the step is read back, and the steps are those
        of synchronous mode."""
        out = 0
        started = 0
        if getattr(self, "frozen", False):
            for slot, done in produced:
                if done:
                    out += 1
                    if tokens is not None:
                        self.sched.feed(slot, tokens[slot])
            return out
        for slot, done in produced:
            if not done:
                continue
            out += 1
            self.made[slot] += 1
            if slot not in self.decoding:
                self.decoding.add(slot)
                started += 1
            if tokens is not None:
                self.sched.feed(slot, tokens[slot])
        for _ in range(started):
            slot = max(self.decoding, key=lambda s: (self.made[s] / self.target[s], -s))
            self.decoding.discard(slot)
            self.sched.finish(slot)
        self.admit_arrivals()
        return out

    def decode_only(self):
        """From here on every step is the decoders alone: the requests mid-prefill are
        finished and nothing arrives or retires (each decoder's lease grows as it goes)."""
        self.frozen = True
        for slot in [s for s in self.target if s not in self.decoding]:
            self.sched.finish(slot)
            del self.target[slot]

    def step(self):
        """One synchronous step: (output tokens, prefill tokens, decodes, timings)."""
        produced, prefill, decodes, tm = self.sched.step()
        out = self.decide([(s, d) for s, _, d in produced], {s: t for s, t, d in produced if d})
        return out, prefill, decodes, tm

    def submit(self):
        """Overlap mode: enqueue the next step and take its decisions at once."""
        info, prefill, decodes = self.sched.submit()
        out = self.decide(info)
        return out, prefill, decodes


def run_steps(wl, ctx, steps, warmup, sync, profile=True, kinds=None):
    """Warm-up steps, then exactly `steps` timed steps. Overlap mode keeps one step
    in flight while the host schedules the next; the pipeline starts empty and is
    drained inside the timed region, so the wall time covers exactly the timed
    steps. -> (elapsed s, output tokens, prefill tokens, decodes, device ms)."""
    if not sync:
        wl.sched.set_overlap(True)

    def run(n, timed):
        tot = [0, 0, 0, 0.0]
        if sync:
            for i in range(n):
                out, pf, dc, tm = wl.step()
                tot[0] += out
                tot[1] += pf
                tot[2] += dc
                tot[3] += tm.device_ms
                if timed and (i + 1) % 50 == 0:
                    print("step %d/%d" % (i + 1, n), file=sys.stderr, flush=True)
            return tot
        flight = [wl.submit()] if n else []
        for i in range(n):
            if i + 1 < n:
                flight.append(wl.submit())
            _, tm = wl.sched.collect()
            out, pf, dc = flight.pop(0)
            tot[0] += out
            tot[1] += pf
            tot[2] += dc
            tot[3] += tm.device_ms
            if timed and (i + 1) % 50 == 0:
                print("step %d/%d" % (i + 1, n), file=sys.stderr, flush=True)
        return tot

    run(warmup, False)
    ctx.sync()
    # HIP events around the attention launch (and the launches of `kinds`) of
    # every 4th layer (each layer's launches do the same work; each record
    # leaves the device idle ~4 us)
    if profile:
        import tgo_amd
        ctx.set_profile_kernels(PROFILE_STRIDE, kinds or (tgo_amd.PROF_ATTN,))
    t0 = time.perf_counter()
    out, pf, dc, dev_ms = run(steps, True)
    ctx.sync()
    elapsed = time.perf_counter() - t0
    return elapsed, out, pf, dc, dev_ms


class SharedPrefixWorkload(Workload):
    """256 decoding sequences that all begin with the same
    2048-token prefix (its 128 pages held once by the prefix pool) followed by a
    unique suffix of U[32, 1024] tokens, plus one arriving request prefilling in
    1024-token chunks at every step. An arrival's prompt is the same prefix plus
    a unique tail of U[1, 4] whole chunks, so the pool shares its prefix and
    each step carries exactly one 1024-token chunk. Output budgets and
    completions as in config 4."""

    def __init__(self, tgo, ctx, seed):
        self.rng = np.random.default_rng(seed)
        self.sched = tgo.Scheduler(ctx, C5_DECODERS + 8, chunk=C5_CHUNK, reserve=512,
                                   max_rows=C5_CHUNK + C5_DECODERS)
        self.target, self.made, self.decoding = {}, {}, set()
        self.V = C5["vocab"]
        self.prefix = [int(t) for t in self.rng.integers(0, self.V, C5_PREFIX)]
        used = C5_PREFIX
        for _ in range(C5_DECODERS):
            n = int(self.rng.integers(32, 1025))
            out = int(self.rng.integers(100, 301))
            prompt = self.prefix + [int(t) for t in self.rng.integers(0, self.V, n)]
            slot = self.sched.admit_prefilled(prompt, int(self.rng.integers(0, self.V)), reserve=out)
            self.target[slot], self.made[slot] = out, int(self.rng.integers(0, out))
            self.decoding.add(slot)
            used += n + out
        self.used_positions = used
        self.contexts = [self.sched.length(s) for s in sorted(self.decoding)]
        self.admit_arrivals()

    def admit_arrivals(self):
        while self.sched.prefilling() < 1:
            tail = C5_CHUNK * int(self.rng.integers(1, 5))
            out = int(self.rng.integers(100, 301))
            prompt = self.prefix + [int(t) for t in self.rng.integers(0, self.V, tail)]
            slot = self.sched.admit(prompt, reserve=out)
            self.target[slot], self.made[slot] = out, 0


def run_c5(args, tgo_amd):
    """BASELINE config 5 through the same Scheduler, with prefix-shared attention."""
    form = 1 if args.form == 3 else args.form  # config 5 is an int8 model
    t_setup = time.perf_counter()
    ctx = tgo_amd.Context(0)
    ctx.set_precision(args.precision)
    ctx.set_cascade(args.cascade)
    ctx.config(C5["layers"], C5["hidden"], C5["heads"], C5["kv_heads"], C5["head_dim"],
               C5["ffn"], C5["vocab"], C5["rms_eps"], C5["rope_theta"], C5["block"])
    # the KV pool before anything else: allocated first in the process, its pages
    # fall in the faster of two placements for attention
    ctx.kv_alloc(C5_POOL)
    ctx.synth_weights(SEED, form, 0.02)
    wl = SharedPrefixWorkload(tgo_amd, ctx, SEED)
    ctx.kv_synth(SEED, 1.0, min(C5_POOL, wl.used_positions + 32 * C5_CHUNK))
    print("setup %.1f s: config 5 weights synthesized, %d decoders admitted on a %d-token "
          "shared prefix (mean context %.0f)" % (time.perf_counter() - t_setup, C5_DECODERS,
          C5_PREFIX, np.mean(wl.contexts)), file=sys.stderr, flush=True)
    elapsed, total_out, total_pf, total_dc, dev_ms = run_steps(wl, ctx, args.steps, args.warmup,
                                                               args.sync)
    attn_ms, attn_bytes, launches = ctx.profile_read()
    ctx.set_profile(False)
    kernels = profile_kernels(wl, ctx, tgo_amd, PROFILE_STEPS, args.sync)
    ctx.close()
    avg_attn_ms = attn_ms / max(launches, 1)
    achieved = (attn_bytes / max(launches, 1)) / (avg_attn_ms * 1e-3) / 1e9
    return {
        "metric": "output tok/s, Qwen3-32B int8 prefix-shared batch, 1 MI355X; paged-attn HBM GB/s",
        "value": round(total_out / elapsed, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * elapsed / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if args.precision == 0 else "f32 (f16 hi+lo operand pairs, 3 MFMAs per product)",
        "data": "synthetic (seeded random-init int8 weights, seeded token ids, synthetic KV for "
                "the initial contexts)",
        "config": {
            "workload": "BASELINE config 5: Qwen3-32B-shaped int8 (64 layers, hidden 5120, 64 q / "
                        "8 kv heads, MLP 25600), 256 decode sequences on one 2048-token shared "
                        "prefix + unique suffixes U[32,1024], one 1024-token prefill chunk per "
                        "step, page 16, f16 KV, greedy, prefix-shared attention " +
                        ("on (groups of >= %d)" % args.cascade if args.cascade else "off"),
            "weight_form": {2: "int4-tgo-g128-asym", 1: "int8", 0: "f16"}.get(form, str(form)),
            "rows_per_step": round((total_pf + total_dc) / args.steps, 1),
            "prefill_tokens_per_step": round(total_pf / args.steps, 1),
            "decodes_per_step": round(total_dc / args.steps, 1),
            "output_tokens": int(total_out),
            "device_ms_per_step": round(dev_ms / args.steps, 3),
            "host_overlap": not args.sync,
        },
        "roofline": {
            "kernel": "attn_kernel + attn_combine_kernel (ragged paged attention, shared "
                      "prefix read once per group)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK, 4),
            "traffic": None,
            "avg_launch_ms": round(avg_attn_ms, 4),
            "algorithmic_bytes_per_launch": round(attn_bytes / max(launches, 1)),
            "launches": launches,
        },
        "cpu_baseline": None,
        "kernels": kernels,
    }


def run_c1(args, tgo_amd):
    """Qwen3-0.6B-shaped, random-init f16 weights N(0, 0.02); one
    continuous-batching step of 3 decoding sequences (contexts 37, 300, 511) plus a
    64-token chunk of a fresh sequence, page 16. The step is built by the library
    Scheduler and replayed through tgohip_step (rewriting its K/V rows with the same
    values is idempotent) with tgohip_step, which waits for the step and reads back the
    greedy tokens: ms_per_step is the synchronous step's latency. The CPU restatement of
    tgo's path steps the same ports."""
    c = C1
    ctx = tgo_amd.Context(0)
    ctx.set_precision(args.precision)
    ctx.config(c["layers"], c["hidden"], c["heads"], c["kv_heads"], c["head_dim"], c["ffn"],
               c["vocab"], c["rms_eps"], c["rope_theta"], c["block"])
    ctx.kv_alloc(C1_POOL)
    ctx.synth_weights(SEED, tgo_amd.FORM_F16, 0.02)
    rng = np.random.default_rng(SEED)
    sched = tgo_amd.Scheduler(ctx, 4, chunk=C1_CHUNK, reserve=16, max_rows=C1_CHUNK + 3)
    for n in C1_CONTEXTS:
        sched.admit_prefilled([int(t) for t in rng.integers(0, c["vocab"], n)],
                              int(rng.integers(0, c["vocab"])), reserve=16)
    sched.admit([int(t) for t in rng.integers(0, c["vocab"], C1_CHUNK)], reserve=16)
    ctx.kv_synth(SEED, 1.0, C1_POOL)
    _, prefill, decodes, _ = sched.step()
    assert (prefill, decodes) == (C1_CHUNK, len(C1_CONTEXTS)), (prefill, decodes)
    st, pages, maxp = sched.last_step()
    members = len(st["lengths"])
    for _ in range(args.warmup):
        ctx.step(st, pages, maxp, want_logits=False)
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ctx.step(st, pages, maxp, want_logits=False)
    ctx.sync()
    el = time.perf_counter() - t0
    ms = 1e3 * el / args.steps
    ctx.close()
    d, f, L, V = c["hidden"], c["ffn"], c["layers"], c["vocab"]
    qw, kw = c["heads"] * 128, c["kv_heads"] * 128
    weights = 2.0 * (L * (d * (qw + 2 * kw) + qw * d + 2 * d * f + f * d) + d * V)
    gbs = weights / (ms * 1e-3) / 1e9
    out = {
        "metric": "step latency and output tok/s, Qwen3-0.6B f16 one continuous-batching step, "
                  "1 MI355X",
        "value": round(members / (ms * 1e-3), 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if args.precision == 0 else "f32 (f16 hi+lo operand pairs)",
        "data": "synthetic (seeded random-init f16 weights, seeded token ids, synthetic KV)",
        "config": {"workload": "BASELINE config 1: Qwen3-0.6B-shaped f16 (28 layers, hidden 1024, "
                               "16 q / 8 kv heads, MLP 3072, vocab 151936); 3 decodes at contexts "
                               "37/300/511 + a 64-token chunk of a fresh sequence, page 16; the "
                               "one step replayed (%d rows, %d members)" % (len(st["ids"]), members)},
        "roofline": {"kernel": "the whole step (weights once: the 28 layers' f16 projections "
                               "and the LM head)",
                     "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK, 4), "traffic": None,
                     "algorithmic_bytes_per_step": round(weights)},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        import oracle
        cpu = oracle.CPUModel(L, d, c["heads"], c["kv_heads"], c["head_dim"], f, V, c["rms_eps"],
                              c["rope_theta"], c["block"], C1_POOL)
        cpu.synth(SEED, tgo_amd.FORM_F16, 0.02)
        cpu.step(st, pages, maxp)  # first touch of its pool and weights
        t0 = time.perf_counter()
        cpu.step(st, pages, maxp)
        cs = time.perf_counter() - t0
        cpu.close()
        out["cpu_baseline"] = dict(value=round(members / cs, 3), unit="tok/s",
                                   cores=int(oracle.lib.orc_num_threads()), kind="port",
                                   sample="the same step (%d rows, all 28 layers) stepped once by "
                                          "the CPU restatement after a first-touch step: %.3f s; "
                                          "KV contents zero" % (len(st["ids"]), cs))
    return out


def kernel_table(ctx, tgo, kinds):
    """Per-launch means of the profiled kernel kinds: duration, algorithmic bytes and flops,
    and the fractions of the HBM and dense f16 MFMA peaks they reach."""
    out = {}
    for k in kinds:
        ms, by, fl, n = ctx.profile_read_kernel(k)
        if not n:
            continue
        avg = ms / n
        gbs = by / n / (avg * 1e-3) / 1e9
        tfs = fl / n / (avg * 1e-3) / 1e12
        out[tgo.PROF_NAMES[k]] = dict(avg_ms=round(avg, 4), launches=n,
                                      bytes=round(by / n), flops=round(fl / n),
                                      gbps=round(gbs, 1), hbm_frac=round(gbs / HBM_PEAK, 4),
                                      tflops=round(tfs, 1), mfma_frac=round(tfs / MFMA_F16_PEAK, 4))
    return out


def profile_kernels(wl, ctx, tgo, steps, sync):
    """`steps` more steps with every kernel kind of every 4th layer bracketed by events
    (not part of any timed figure)."""
    kinds = (tgo.PROF_ATTN, tgo.PROF_QKV, tgo.PROF_O, tgo.PROF_GATEUP, tgo.PROF_DOWN,
             tgo.PROF_LMHEAD)
    ctx.set_profile_kernels(PROFILE_STRIDE, kinds)
    run_steps(wl, ctx, steps, 0, sync, profile=False)
    table = kernel_table(ctx, tgo, kinds)
    ctx.set_profile(False)
    return table


def step_bytes(c, form, rows, members, attn_bytes_per_launch, precision):
    """Algorithmic HBM bytes of one step: every weight once (the layers' projections, the
    LM head, the embedding rows gathered), the KV the attention reads (from the profiled
    launches, less their q in / out) and writes, and the logits written."""
    d, f, V, L = c["hidden"], c["ffn"], c["vocab"], c["layers"]
    qw, kw = c["heads"] * 128, c["kv_heads"] * 128
    per_weight = {3: 0.5 + 2 / 32, 2: 0.5 + 4 / 128, 1: 1 + 2 / 32, 0: 2.0}[form]
    layer_w = (d * (qw + 2 * kw) + qw * d + 2 * d * f + f * d) * per_weight
    weights = L * layer_w + d * V * per_weight + rows * d * (1 + 2 / 32)
    q_io = rows * c["heads"] * 128 * (4 if precision == 0 else 8)  # q in, out
    kv_read = L * (attn_bytes_per_launch - q_io)
    kv_write = L * rows * kw * 2 * 2
    logits = members * V * 4
    total = weights + kv_read + kv_write + logits
    return total, dict(weights=round(weights), kv_read=round(kv_read), kv_write=round(kv_write),
                       logits=round(logits))


def recorded_mfma():
    """MFMA counters per projection kernel on this workload (rocprofv3 --pmc), as profiles/
    records them: dense f16 MFMA flops executed per dispatch (SQ_INSTS_VALU_MFMA_MOPS_F16 x
    512) over the dispatch's duration, and the MFMA busy fraction
    (SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x SIMDs))."""
    path = os.path.join(ROOT, "profiles", "gemm_mfma_c4_pmc.txt")
    if not os.path.exists(path):
        return None
    out = {}
    for line in open(path):
        if line.startswith("mfma "):
            _, step, name, tflops, frac, busy = line.split()
            out.setdefault(step, {})[name] = dict(tflops=float(tflops), mfma_frac=float(frac),
                                                  mfma_busy=float(busy))
    return out or None


def recorded_traffic():
    """HBM bytes per attention launch measured with rocprofv3 --pmc on this workload
    (FETCH_SIZE + WRITE_SIZE, each scaled by a copy probe), as profiles/ records it."""
    path = os.path.join(ROOT, "profiles", "attn_kernel_c4_pmc.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch attn_kernel:"):
            return float(line.split(":")[1])
    return None


def recorded_proj_traffic(step, proj):
    """HBM bytes per dispatch of one projection (FETCH_SIZE + WRITE_SIZE, each scaled by a
    copy probe) on this workload, as profiles/ records it -> (fetch, write) or None."""
    path = os.path.join(ROOT, "profiles", "gemm_traffic_c4_pmc.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        f = line.split()
        if len(f) == 5 and f[0] == "traffic" and f[1] == step and f[2] == proj:
            return float(f[3]), float(f[4])
    return None


def cpu_baseline(st, pages, max_pages, out_tokens, form):
    """tgo's CPU path restated (oracle/, OpenMP) on one timed step: the step with 1
    and 2 layers, the per-layer time extrapolated to 36 layers."""
    import oracle
    c = C4
    m = oracle.CPUModel(2, c["hidden"], c["heads"], c["kv_heads"], c["head_dim"], c["ffn"],
                        c["vocab"], c["rms_eps"], c["rope_theta"], c["block"], POOL)
    try:
        m.synth(SEED, form, 0.02, 2)
        t = time.perf_counter()
        m.step(st, pages, max_pages, layers=1)
        t1 = time.perf_counter() - t
        t = time.perf_counter()
        m.step(st, pages, max_pages, layers=2)
        t2 = time.perf_counter() - t
    finally:
        m.close()
    per_layer = max(t2 - t1, 1e-9)
    full = t1 + (c["layers"] - 1) * per_layer
    return dict(value=out_tokens / full, unit="tok/s", cores=int(oracle.lib.orc_num_threads()),
                kind="port",
                sample=("one timed step (%d rows, %d sequences) of the same workload run by the "
                        "CPU restatement with 1 layer (%.1f s) and 2 layers (%.1f s); step time "
                        "extrapolated to 36 layers = %.1f s; KV contents zero, weights the same "
                        "synthesized int4" % (len(st["ids"]), len(st["lengths"]), t1, t2, full)),
                seconds=t1 + t2)


def run_decode_phase(wl, ctx, tgo, args):
    """The decode-dominated step the north-star target is judged on: the same 128
    decoders (their contexts grown by the timed steps) with no prefill chunk, 128 rows per
    step. Timed like the headline (warm-up, then exactly decode_steps steps, attention
    launches of every 4th layer bracketed by events); then a few steps with every kernel
    timed. Whole-step HBM fraction = algorithmic bytes of a step (weights once, KV read and
    written, logits) / the step's wall time / 8 TB/s."""
    wl.decode_only()
    el, out, pf, dc, dev_ms = run_steps(wl, ctx, args.decode_steps, 5, args.sync)
    assert pf == 0 and dc == DECODERS * args.decode_steps, (pf, dc)
    attn_ms, attn_bytes, launches = ctx.profile_read()
    ctx.set_profile(False)
    kernels = profile_kernels(wl, ctx, tgo, PROFILE_STEPS, args.sync)
    ms = 1e3 * el / args.decode_steps
    rows = DECODERS
    # logits are written for the members that worked only (the 128 decoders)
    total, parts = step_bytes(C4, args.form, rows, DECODERS, attn_bytes / max(launches, 1),
                              args.precision)
    gbs = total / (ms * 1e-3) / 1e9
    avg_attn = attn_ms / max(launches, 1)
    attn_gbs = attn_bytes / max(launches, 1) / (avg_attn * 1e-3) / 1e9
    return dict(
        workload="the 128 decoders of the headline run continuing alone (no prefill chunk): "
                 "128 rows per step, contexts lognormal median 1024 grown by the steps before",
        steps=args.decode_steps, ms_per_step=round(ms, 3), tok_per_s=round(out / el, 1),
        device_ms_per_step=round(dev_ms / args.decode_steps, 3),
        hbm_bytes_per_step=round(total), bytes=parts, hbm_gbps=round(gbs, 1),
        hbm_frac=round(gbs / HBM_PEAK, 4),
        attention=dict(avg_launch_ms=round(avg_attn, 4), gbps=round(attn_gbs, 1),
                       frac=round(attn_gbs / HBM_PEAK, 4), launches=launches),
        kernels=kernels)


def run_fast_leg(wl, ctx, tgo, args, what):
    """`fast_steps` more steps of the same workload with f16 operands (precision 0: one
    MFMA per product, activations, weights and probabilities rounded to f16), then back to
    tgo's arithmetic. Mixed steps go on with arrivals and completions; decode-only steps
    follow the decode phase."""
    ctx.set_precision(0)
    el, out, pf, dc, dev_ms = run_steps(wl, ctx, args.fast_steps, 3, args.sync, profile=False)
    ctx.set_precision(args.precision)
    r = dict(steps=args.fast_steps, ms_per_step=round(1e3 * el / args.fast_steps, 3),
             tok_per_s=round(out / el, 1))
    if what == "mixed":
        r["note"] = ("precision 0 (f16 operands): faster, but its logits drift from tgo's CPU "
                     "path with depth (largest error 5.7e-3 of the row's largest logit after 36 "
                     "layers, tests/test_depth_gpu.py) past the 2e-3 bound the headline's "
                     "arithmetic meets")
    return r


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py: this build measures one MI355X; --gpus %d is not supported (the path "
              "would shard attention by sequence and the projections by column/row with RCCL)"
              % args.gpus, file=sys.stderr)
        sys.exit(2)
    if args.copy_probe_mib:
        copy_probe(args.copy_probe_mib)
    import tgo_amd
    if args.config == "c5":
        print(json.dumps(run_c5(args, tgo_amd)), flush=True)
        return
    if args.config == "c1":
        print(json.dumps(run_c1(args, tgo_amd)), flush=True)
        return
    t_setup = time.perf_counter()
    ctx = tgo_amd.Context(0)
    # the box's achievable peaks, before any pool or weight is allocated
    ach = achievable_peaks(ctx) if args.phase == "both" else None
    ctx.set_precision(args.precision)
    ctx.config(C4["layers"], C4["hidden"], C4["heads"], C4["kv_heads"], C4["head_dim"],
               C4["ffn"], C4["vocab"], C4["rms_eps"], C4["rope_theta"], C4["block"])
    # the KV pool before anything else: allocated first in the process, its pages
    # fall in the faster of two placements for attention (8 of 8 trials, against
    # 5 of 8 when it followed the weights)
    ctx.kv_alloc(POOL)
    ctx.synth_weights(SEED, args.form, 0.02)
    wl = Workload(tgo_amd, ctx, SEED)
    ctx.kv_synth(SEED, 1.0, min(POOL, wl.used_positions + 64 * CHUNK))
    setup_s = time.perf_counter() - t_setup
    print("setup %.1f s: weights synthesized, %d decoders admitted (mean context %.0f)" %
          (setup_s, DECODERS, np.mean([x for x in wl.contexts if x > 0])), file=sys.stderr,
          flush=True)

    if args.phase == "decode":
        decode = run_decode_phase(wl, ctx, tgo_amd, args)
        ctx.close()
        print(json.dumps(dict(phase="decode", decode_step=decode)), flush=True)
        return
    # the timed steps bracket attention and the SwiGLU gate/up (the step's largest
    # kernel) of every 4th layer with events: the line's two roofline objects
    elapsed, total_out, total_pf, total_dc, dev_ms = run_steps(
        wl, ctx, args.steps, args.warmup, args.sync,
        kinds=(tgo_amd.PROF_ATTN, tgo_amd.PROF_GATEUP))
    attn_ms, attn_bytes, launches = ctx.profile_read()
    gu_ms, gu_bytes, gu_flops, gu_n = ctx.profile_read_kernel(tgo_amd.PROF_GATEUP)
    ctx.set_profile(False)
    last_st, last_pages, maxp = wl.sched.last_step()
    # the CPU leg is charged the mean output tokens of a timed step
    last_out = total_out / args.steps
    mixed_kernels = profile_kernels(wl, ctx, tgo_amd, PROFILE_STEPS, args.sync)
    fast = None
    if args.fast_steps and args.precision == 1 and args.phase == "both":
        fast = run_fast_leg(wl, ctx, tgo_amd, args, "mixed")
    decode = None
    if args.decode_steps and args.phase == "both":
        decode = run_decode_phase(wl, ctx, tgo_amd, args)
        if fast:
            fast["decode_step"] = run_fast_leg(wl, ctx, tgo_amd, args, "decode")

    avg_attn_ms = attn_ms / max(launches, 1)
    achieved = (attn_bytes / max(launches, 1)) / (avg_attn_ms * 1e-3) / 1e9
    avg_gu_ms = gu_ms / max(gu_n, 1)
    gu_tflops = (gu_flops / max(gu_n, 1)) / (avg_gu_ms * 1e-3) / 1e12
    # the committed counters were taken at the default arithmetic and weight form only
    gu_traffic = recorded_proj_traffic("mixed", "gateup") \
        if args.precision == 1 and args.form == tgo_amd.FORM_I4_SYM else None
    # tgo's arithmetic: symmetric int4 factors its group scale out (activation
    # hi.code + lo.code, the scale applied in f32); the other forms multiply
    # the exact dequantized weight's hi and lo parts (hi.hi + lo.hi + hi.lo)
    mfma_per_product = 1 if args.precision == 0 else (2 if args.form == 3 else 3)
    rows_per_step = (total_pf + total_dc) / args.steps
    result = {
        "metric": "output tok/s, Qwen3-8B int4 ragged batch, 1 MI355X; paged-attn HBM GB/s",
        "value": round(total_out / elapsed, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * elapsed / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if args.precision == 0 else (
            "f32 (f16 hi+lo activation pairs times the exact int4 codes, 2 MFMAs per product, "
            "group scale applied in f32)" if args.form == 3 else
            "f32 (f16 hi+lo operand pairs, 3 MFMAs per product)"),
        "data": "synthetic (seeded random-init int4 weights, seeded token ids, synthetic KV for "
                "the initial contexts)",
        "config": {
            "workload": "BASELINE config 4: Qwen3-8B-shaped int4 (symmetric g32-K pack), 128 "
                        "decode sequences (contexts lognormal median 1024, sigma 1.0, clipped "
                        "[16,8192]) + 2 prefill chunks of 512 per step, page 16, f16 KV, greedy, "
                        "seeded arrivals/completions",
            "weight_form": {3: "int4-sym-g32K", 2: "int4-tgo-g128-asym", 1: "int8", 0: "f16"}[args.form],
            "rows_per_step": round(rows_per_step, 1),
            "prefill_tokens_per_step": round(total_pf / args.steps, 1),
            "decodes_per_step": round(total_dc / args.steps, 1),
            "output_tokens": int(total_out),
            "device_ms_per_step": round(dev_ms / args.steps, 3),
            "host_overlap": not args.sync,
        },
        "roofline": {
            "kernel": "gemm_pipe_kernel, the SwiGLU gate/up projection (the step's largest "
                      "kernel), %d rows" % round(rows_per_step),
            "bound": "mfma",
            "achieved": round(gu_tflops, 1),
            "peak": MFMA_F16_PEAK,
            "unit": "TFLOP/s",
            "frac": round(gu_tflops / MFMA_F16_PEAK, 4),
            "traffic": round(sum(gu_traffic)) if gu_traffic else None,
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE then WRITE_SIZE over 2 steps of this "
                              "workload at this arithmetic, scaled by a 1 GiB copy probe "
                              "(profiles/gemm_traffic_c4_pmc.txt)" if gu_traffic else None,
            "algorithmic_bytes_per_launch": round(gu_bytes / max(gu_n, 1)),
            "flops_per_launch": round(gu_flops / max(gu_n, 1)),
            "flops_counted": "algorithmic, 2*M*K*N; the kernel executes %d f16 MFMAs per "
                             "product (%s)" % (mfma_per_product, {
                                 3: "activation hi.weight hi + lo.hi + hi.lo",
                                 2: "activation hi.code + lo.code into a per-group sum, "
                                    "times the group's scale in f32",
                                 1: "f16 operands"}[mfma_per_product]),
            "executed_mfma_frac": round(mfma_per_product * gu_tflops / MFMA_F16_PEAK, 4),
            "avg_launch_ms": round(avg_gu_ms, 4),
            "launches": gu_n,
        },
        "roofline_attention": {
            "kernel": "attn_kernel + attn_combine_kernel (ragged paged attention)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK, 4),
            "traffic": recorded_traffic(),
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE then WRITE_SIZE over the first 3 "
                              "steps of this workload, scaled by a 1 GiB copy probe "
                              "(profiles/attn_kernel_c4_pmc.txt)",
            "avg_launch_ms": round(avg_attn_ms, 4),
            "algorithmic_bytes_per_launch": round(attn_bytes / max(launches, 1)),
            "launches": launches,
        },
        "cpu_baseline": None,
        "kernels": mixed_kernels,
        "decode_step": decode,
        "fast_path": fast,
        "mfma_counters": recorded_mfma()
        if args.precision == 1 and args.form == tgo_amd.FORM_I4_SYM else None,
    }
    ctx.close()
    if ach:
        result["achievable"] = ach
        result["roofline_attention"]["frac_of_achievable_read"] = round(achieved / ach["read_gbps"], 4)
        result["roofline"]["frac_of_achievable_mfma"] = round(gu_tflops / ach["mfma_f16_tflops"], 4)
        if decode:
            decode["hbm_frac_of_achievable_read"] = round(decode["hbm_gbps"] / ach["read_gbps"], 4)
    if not args.no_cpu:
        cb = cpu_baseline(last_st, last_pages, maxp, last_out, args.form)
        cb.pop("seconds")
        result["cpu_baseline"] = cb
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
