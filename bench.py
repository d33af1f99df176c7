#!/usr/bin/env python3
"""Decode-attention benchmark on one MI355X, through the C ABI.

Workload (default): BASELINE config 4, the headline roofline case -
Qwen3-0.6B-shape decode attention, 256 independent sequences each with 8192
cached positions plus the new token, 28 layers, 16 q / 8 KV heads,
head_dim 128, NEOX RoPE theta 1e6, Q8_0 KV (~128 GB resident in HBM).

One step = for every sequence and layer: RoPE(q, k), append k/v at pos,
attention over pos+1 positions, output over q.  The timed step is
layer-serial (one g2b_attn_layers call per layer: the decode kernel - RoPE,
append, attention - and, where the schedule splits a sequence, the combine
launch that merges the split partials), as a real model's layer loop would
run it; a one-call-for-all-layers variant is reported beside it.  Inputs
are synthetic, seeded, generated on the device (KV prefill through the same
RoPE + append arithmetic) and resident in HBM before timing starts.  The q
buffer is restored from a pristine copy at the start of each step (that
0.1% of traffic is inside the timed region).

Bytes per step are algorithmic, as BASELINE states them:
  sum over seq, layer of (pos+1)*2*row + 2*row + 4*(2*nq + 2*nkv).

Every config (the headline, then c1, c2, c3, c5 under all_configs) reports
the same block: the layer-serial step, its dominant decode kernel against
the HBM roofline (HIP-event launch time; HBM traffic from the committed
rocprofv3 summary profiles/traffic_<kernel>_<config>.json), the all-layers call, the
CPU baseline - the C99 oracle (a restatement of the reference path, built
with the reference flags) on the same KV bytes and inputs, mode A one thread
over sequences in turn, mode B OpenMP over sequences - and a full-size
parity sample (the oracle's outputs and appended rows against the GPU's,
and two units in float64).  rank 0 prints one JSON line.
"""
from __future__ import annotations

import argparse
import collections
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from gguf2bin_amd import attn, hip  # noqa: E402

METRIC = "decode-attention KV-read GB/s (% of HBM peak) + us/step, Qwen3-0.6B shape"
HBM_PEAK_GBPS = 8000.0
# the weight copies one GEMV measurement cycles through (more than MI355X's
# 256 MB last-level cache holds)
GEMV_COLD_BYTES = 1 << 30
Q3, LL = attn.ARCH_QWEN3, attn.ARCH_LLAMA

# name: (shape, n_seq, (ctx_lo, ctx_hi) cached positions, K-row x8 probability, description)
CONFIGS = {
    "c1": (attn.Shape(28, 16, 8, 128, 1e6, Q3, False), 1, (2048, 2048), 0.0,
           "Qwen3-0.6B shape, 1 seq, F32 KV, ctx 2048+1"),
    "c2": (attn.Shape(28, 16, 8, 128, 1e6, Q3, True), 1, (8192, 8192), 0.0,
           "Qwen3-0.6B shape, 1 seq, Q8_0 KV, ctx 8192+1"),
    "c3": (attn.Shape(30, 9, 3, 64, 1e5, LL, False), 64, (256, 2048), 0.0,
           "SmolLM2-135M shape, 64 seq, F32 KV, ctx U[256,2048]"),
    "c4": (attn.Shape(28, 16, 8, 128, 1e6, Q3, True), 256, (8192, 8192), 0.0,
           "Qwen3-0.6B shape, 256 seq, Q8_0 KV, ctx 8192+1 (~128 GB KV)"),
    "c5": (attn.Shape(32, 32, 8, 128, 5e5, LL, True), 32, (16384, 32767), 0.01,
           "Llama-3-8B shape, 32 seq, Q8_0 KV, ctx U[16384,32767], 1% K rows x8"),
}


def log(msg: str):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def splitmix_uniform(seed: int, n: int) -> np.ndarray:
    """n uniforms in (0,1] from SplitMix64 (same generator as the fills)."""
    m = (1 << 64) - 1
    out = np.empty(n)
    s = seed & m
    for i in range(n):
        s = (s + 0x9E3779B97F4A7C15) & m
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
        z ^= z >> 31
        out[i] = ((z >> 11) + 1) * (1.0 / 9007199254740992.0)
    return out


def norm_ppf(p: float) -> float:
    from statistics import NormalDist
    return float(NormalDist().inv_cdf(p))


def row_bytes(s: attn.Shape) -> int:
    return attn.kv_row_bytes(s)


def step_bytes(s: attn.Shape, poss) -> int:
    rb = row_bytes(s)
    per = sum((p + 1) * 2 * rb + 2 * rb + 4 * (2 * s.nq + 2 * s.nkv) for p in poss)
    return per * s.n_layers


def launch_bytes(s: attn.Shape, poss, layers_per_launch: int) -> int:
    """Algorithmic bytes of one k_layer launch: the step's per-layer bytes
    (KV read of positions 0..pos, the appended rows, q/out/k/v) for every
    layer the launch covers."""
    return step_bytes(s, poss) // s.n_layers * layers_per_launch


def source_digest() -> str:
    """sha256 (first 16 hex digits) of the library's device and host sources
    (gguf2bin_amd/csrc, gguf2bin_amd/host, include): the build a committed
    profile was measured on records it, and a run compares it with its own
    (the GPU box gets the tree without its git history)."""
    import hashlib
    h = hashlib.sha256()
    for d in ("gguf2bin_amd/csrc", "gguf2bin_amd/host", "include"):
        base = os.path.join(ROOT, d)
        for name in sorted(os.listdir(base)):
            if name.endswith((".h", ".hip", ".c")):
                h.update(f"{d}/{name}\0".encode())
                with open(os.path.join(base, name), "rb") as f:
                    h.update(f.read())
    return h.hexdigest()[:16]


def load_traffic(workload: str, kernel: str):
    """HBM bytes per launch of the workload's decode kernel, measured with
    rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE) and scaled by a copy kernel of
    known size, when that summary (profiles/traffic_<kernel>_<workload>.json)
    has been committed."""
    p = os.path.join(ROOT, "profiles", f"traffic_{kernel}_{workload}.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f)


# CPU sample of each config: (sequences run in turn on one thread, sequences
# over all host threads).  c1/c2 hold one sequence: the whole step, both
# modes one thread (the reference attention is single-threaded and mode B
# parallelises over sequences only).
CPU_SAMPLE = {"c1": (1, 1), "c2": (1, 1), "c3": (8, 64), "c4": (4, 32), "c5": (1, 8)}


class Workload:
    """One config's KV caches (filled on the device), inputs and step functions."""

    def __init__(self, name: str, args, n_seq_override: int = 0):
        self.name = name
        shape, n_seq, (lo, hi), p_scale, desc = CONFIGS[name]
        if n_seq_override:
            n_seq = n_seq_override
        self.shape, self.n_seq, self.desc = shape, n_seq, desc
        L, nq, nkv = shape.n_layers, shape.nq, shape.nkv
        if lo == hi:
            poss = [lo] * n_seq
        else:
            u = splitmix_uniform(args.seed ^ 0xC7C7, n_seq)
            poss = [int(lo + min(int(x * (hi - lo + 1)), hi - lo)) for x in u]
        self.poss, self.caps = poss, [p + 1 for p in poss]
        thr = norm_ppf(1.0 - p_scale) if p_scale > 0 else float("inf")
        kv_total = sum(2 * attn.kv_bytes(shape, c) for c in self.caps)
        log(f"{name}: {desc}; n_seq={n_seq}, KV {kv_total / 1e9:.2f} GB")
        self.ctx = ctx = attn.Context(shape)
        ctx.tune(args.split, args.chunk, args.stage, args.piece)
        ctx.tune_kernel(args.kernel)
        t0 = time.perf_counter()
        self.kvs = [ctx.kv_alloc(c) for c in self.caps]
        for i, (p, c) in enumerate(zip(poss, self.caps)):
            k, v = self.kvs[i]
            ctx.synth_fill_kv(k, v, c, 0, L, 0, p, args.seed, i, thr)
            if i % 32 == 31:
                ctx.sync()
                log(f"filled {i + 1}/{n_seq} sequences ({time.perf_counter() - t0:.1f}s)")
        ctx.sync()
        self.t_fill = time.perf_counter() - t0
        log(f"KV fill done in {self.t_fill:.1f}s")
        self.nQ, self.nK = L * n_seq * nq, L * n_seq * nkv
        self.q0 = hip.DeviceBuffer(self.nQ * 4)
        self.qw = hip.DeviceBuffer(self.nQ * 4)
        self.kb = hip.DeviceBuffer(self.nK * 4)
        self.vb = hip.DeviceBuffer(self.nK * 4)
        ctx.synth_normal(self.q0.ptr, self.nQ, attn.stream_seed(args.seed, 0, 0, 2))
        ctx.synth_normal(self.kb.ptr, self.nK, attn.stream_seed(args.seed, 0, 0, 3))
        ctx.synth_normal(self.vb.ptr, self.nK, attn.stream_seed(args.seed, 0, 0, 4))
        ctx.batch_begin([(p, c, k, v) for p, c, (k, v) in zip(poss, self.caps, self.kvs)])
        ctx.sync()
        self.bytes_per_step = step_bytes(shape, poss)

    def step_layer_serial(self):
        s, ctx, n = self.shape, self.ctx, self.n_seq
        ctx.synth_copy(self.qw.ptr, self.q0.ptr, self.nQ * 4)
        for layer in range(s.n_layers):
            ctx.attn_layers(layer, 1, self.qw.ptr + layer * n * s.nq * 4,
                            self.kb.ptr + layer * n * s.nkv * 4,
                            self.vb.ptr + layer * n * s.nkv * 4)

    def step_fused(self):
        self.ctx.synth_copy(self.qw.ptr, self.q0.ptr, self.nQ * 4)
        self.ctx.attn_layers(0, self.shape.n_layers, self.qw.ptr, self.kb.ptr, self.vb.ptr)

    def timed(self, step, steps, warmup):
        """(event ms per step, host ms per step, decode-kernel ms summed, launches).
        The step time comes from a pass with nothing but the step on the
        stream; the decode kernels' own durations from a second pass of the
        same steps with a pair of events around every decode launch (which
        would otherwise add their own gaps to the step)."""
        ctx = self.ctx
        for _ in range(warmup):
            step()
        ctx.sync()
        e0, e1 = hip.Event(), hip.Event()
        h0 = time.perf_counter()
        e0.record(ctx.stream)
        for _ in range(steps):
            step()
        e1.record(ctx.stream)
        e1.synchronize()
        wall = time.perf_counter() - h0
        ctx.profile(True)
        ctx.profile_read()
        for _ in range(steps):
            step()
        dms, nlaunch = ctx.profile_read()
        ctx.profile(False)
        return e0.elapsed_ms(e1) / steps, wall / steps * 1e3, dms, nlaunch

    def summary(self, args, steps, warmup, cpu_min_s, fused=True, cpu=True):
        """Every figure of this config: the layer-serial step (us, GB/s, % of
        peak), its dominant decode kernel against the HBM roofline (with the
        committed rocprofv3 traffic), the all-layers-in-one-call step, the
        CPU baseline in both modes and the full-size parity sample.  Leaves
        the layer-serial outputs in qw."""
        ms, wall_ms, dms, dn = self.timed(self.step_layer_serial, steps, warmup)
        sched = self.ctx.last_schedule()
        sb, L = self.bytes_per_step, self.shape.n_layers
        gbps = sb / (ms * 1e-3) / 1e9
        dec_ms = dms / max(dn, 1)
        per_launch = launch_bytes(self.shape, self.poss, 1)
        dec_gbps = per_launch / (dec_ms * 1e-3) / 1e9
        log(f"{self.name}: layer-serial {ms * 1e3:.1f} us/step (host {wall_ms * 1e3:.1f}), "
            f"{gbps:.1f} GB/s, {100 * gbps / HBM_PEAK_GBPS:.1f}% of HBM peak; decode kernel "
            f"{dn} launches, avg {dec_ms * 1e3:.2f} us, {dec_gbps:.1f} GB/s")
        traffic = load_traffic(self.name, sched["kernel"])
        # the committed traffic counts only where they were measured on this
        # kernel instance and these sources
        digest = source_digest()
        current = bool(traffic) and traffic.get("kernel") == sched["variant"] and \
            traffic.get("source_digest") == digest
        roof = {"bound": "hbm", "kernel": sched["variant"],
                "achieved": round(dec_gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(dec_gbps / HBM_PEAK_GBPS, 4), "bytes_per_launch": per_launch,
                "avg_launch_us": round(dec_ms * 1e3, 3),
                "traffic": traffic.get("hbm_bytes_per_launch") if current else None,
                "source_digest": digest}
        if traffic:
            roof["traffic_source"] = traffic.get("source")
            roof["traffic_profile"] = {"kernel": traffic.get("kernel"),
                                       "commit": traffic.get("commit"),
                                       "source_digest": traffic.get("source_digest"),
                                       "matches_this_run": current}
            if current:
                roof["traffic_over_algorithmic"] = traffic.get("traffic_over_algorithmic")
        out = {"workload": self.desc, "n_seq": self.n_seq,
               "ctx_min": min(self.poss), "ctx_max": max(self.poss),
               "us_per_step": round(ms * 1e3, 2), "GBps": round(gbps, 2),
               "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
               "bytes_per_step": sb, "kv_fill_s": round(self.t_fill, 2),
               "step": "layer-serial: one g2b_attn_layers call per layer",
               "schedule": sched, "roofline": roof}
        if fused:
            fms, _, fdms, fdn = self.timed(self.step_fused, steps, 1)
            out["all_layers_one_call"] = {
                "us_per_step": round(fms * 1e3, 2), "GBps": round(sb / (fms * 1e-3) / 1e9, 2),
                "pct_hbm_peak": round(100 * sb / (fms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 2),
                "decode_kernel_avg_us": round(fdms / max(fdn, 1) * 1e3, 2),
                "schedule": self.ctx.last_schedule()}
            log(f"{self.name}: all layers in one call {fms * 1e3:.1f} us/step, "
                f"{out['all_layers_one_call']['GBps']} GB/s")
        # the layer-serial outputs, for the parity sample
        self.step_layer_serial()
        self.ctx.sync()
        if cpu:
            na, nb = CPU_SAMPLE.get(self.name, (1, 1))
            if args.cpu_seq_a:
                na = args.cpu_seq_a
            if args.cpu_seq_b:
                nb = args.cpu_seq_b
            out["cpu_baseline"], out["parity_full_size"] = cpu_leg(self, na, nb, cpu_min_s)
            out["gpu_over_cpu"] = round(gbps / out["cpu_baseline"]["value"], 1)
        return out

    def close(self):
        for k, v in self.kvs:
            self.ctx.kv_free(k, v)
        for b in (self.q0, self.qw, self.kb, self.vb):
            b.free()
        self.ctx.close()


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c4", choices=sorted(CONFIGS))
    ap.add_argument("--n-seq", type=int, default=0, help="override the sequence count")
    ap.add_argument("--seed", type=int, default=20241201)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline and parity legs")
    ap.add_argument("--no-fused", action="store_true", help="skip the all-layers-in-one-call run")
    ap.add_argument("--no-gemv", action="store_true", help="skip the weight-GEMV measurement")
    ap.add_argument("--no-model", action="store_true",
                    help="skip the whole-decode-step (model_forward) measurement")
    ap.add_argument("--no-others", action="store_true",
                    help="skip the other BASELINE configs (reported under all_configs)")
    ap.add_argument("--cpu-seq-a", type=int, default=0,
                    help="sequences in the 1-thread sample (0 = the config's default)")
    ap.add_argument("--cpu-seq-b", type=int, default=0,
                    help="sequences in the all-threads sample (0 = the config's default)")
    ap.add_argument("--cpu-min-s", type=float, default=8.0,
                    help="repeat each CPU sample of the headline config until it has run this "
                         "long (the other configs: a third of it)")
    ap.add_argument("--split", type=int, default=0, help="static split length (0 = automatic)")
    ap.add_argument("--chunk", type=int, default=0, help="Q8 elements per lane (0 = auto)")
    ap.add_argument("--stage", type=int, default=0, choices=(-1, 0, 1, 2),
                    help="KV row path: -1 per-lane HBM loads, 1 global_load_lds chunks, "
                         "2 register-pipelined chunks through LDS (0 = automatic)")
    ap.add_argument("--piece", type=int, default=0,
                    help="schedule: -1 static splits, >0 work-queue piece length (0 = automatic)")
    ap.add_argument("--kernel", type=int, default=0, choices=(0, 1, 2, 3),
                    help="decode kernel: 0 automatic, 1 k_layer only, 2 k_tiles where it "
                         "applies, 3 spanned k_short wherever it applies")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="before timing, run one plain copy kernel of this many MiB (a "
                         "known-size reference for rocprofv3 byte counters)")
    ap.add_argument("--sweep-splits", default="", help="comma list: time layer-serial per split")
    ap.add_argument("--sweep-variants", default="",
                    help="semicolon list of split,chunk,stage,piece: time layer-serial and fused")
    ap.add_argument("--model-only", action="store_true",
                    help="only the whole-decode-step leg (model_forward), printed as its JSON")
    ap.add_argument("--phases", action="store_true",
                    help="only the per-phase breakdown of the config's layer-serial launches, "
                         "from the phase-stamp library (make -C gguf2bin_amd stamps), printed "
                         "as its JSON")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only the weight-GEMV leg (with --calibrate-copy first when given), "
                         "printed as its JSON")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(sharding across GPUs is designed, not built)", file=sys.stderr)
        sys.exit(2)
    if hip.device_count() < 1:
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.phases:  # (before anything loads the library)
        attn.LIBPATH = attn.STAMPS_LIBPATH
    hip.set_device(0)
    if args.phases:
        w = Workload(args.config, args, args.n_seq)
        print(json.dumps({"phases": phases_leg(w, args.steps, args.warmup)}), flush=True)
        w.close()
        return
    if args.model_only:
        print(json.dumps({"model_forward": model_leg(args)}), flush=True)
        return
    if args.gemv_only:
        if args.calibrate_copy:
            cctx = attn.Context(attn.Shape(1, 2, 1, 64, 1e4, attn.ARCH_QWEN3, False))
            nb = args.calibrate_copy << 20
            src, dst = hip.DeviceBuffer(nb), hip.DeviceBuffer(nb)
            cctx.synth_copy(dst.ptr, src.ptr, nb)
            cctx.sync()
            src.free()
            dst.free()
            cctx.close()
            log(f"calibration copy of {args.calibrate_copy} MiB done")
        print(json.dumps({"gemv": gemv_leg(args)}), flush=True)
        return

    w = Workload(args.config, args, args.n_seq)
    ctx, shape, poss = w.ctx, w.shape, w.poss
    if args.calibrate_copy:
        nb = args.calibrate_copy << 20
        src, dst = hip.DeviceBuffer(nb), hip.DeviceBuffer(nb)
        ctx.synth_copy(dst.ptr, src.ptr, nb)
        ctx.sync()
        src.free()
        dst.free()
        log(f"calibration copy of {args.calibrate_copy} MiB done")

    sb = w.bytes_per_step
    if args.sweep_splits:
        for sl in [int(x) for x in args.sweep_splits.split(",")]:
            ctx.tune(sl, args.chunk, args.stage, -1)
            sms, _, sd, sn = w.timed(w.step_layer_serial, max(3, args.steps // 2), 1)
            log(f"split {sl}: {sms * 1e3:.1f} us/step, {sb / sms / 1e6:.1f} GB/s, "
                f"decode kernel avg {sd / max(sn, 1) * 1e3:.1f} us")
        ctx.tune(args.split, args.chunk, args.stage, args.piece)
    if args.sweep_variants:
        for v in args.sweep_variants.split(";"):
            sl, ch, st, pc = [int(x) for x in v.split(",")]
            ctx.tune(sl, ch, st, pc)
            sms, _, sd, sn = w.timed(w.step_layer_serial, max(3, args.steps // 2), 1)
            fms, _, fd, fn = w.timed(w.step_fused, max(3, args.steps // 2), 1)
            log(f"variant split={sl} chunk={ch} stage={st} piece={pc}: layer-serial "
                f"{sms * 1e3:.1f} us/step ({sb / sms / 1e6:.1f} GB/s, decode kernel "
                f"{sd / max(sn, 1) * 1e3:.1f} us), fused {fms * 1e3:.1f} us/step "
                f"({sb / fms / 1e6:.1f} GB/s)")
        ctx.tune(args.split, args.chunk, args.stage, args.piece)

    head = w.summary(args, args.steps, args.warmup, args.cpu_min_s, fused=not args.no_fused,
                     cpu=not args.no_cpu)
    w.close()

    others = None
    if not args.no_others:
        others = {}
        for name in sorted(CONFIGS):
            if name == args.config:
                continue
            o = Workload(name, args)
            others[name] = o.summary(args, max(5, args.steps // 2), 2, args.cpu_min_s / 3,
                                     cpu=not args.no_cpu)
            o.close()

    gemv = None if args.no_gemv else gemv_leg(args)
    model = None if args.no_model else model_leg(args)

    ms = head["us_per_step"] * 1e-3
    gbps = head["GBps"]
    line = {
        "metric": METRIC, "value": gbps, "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"{args.config}: {w.desc}", "n_seq": w.n_seq,
                   "ctx_min": min(poss), "ctx_max": max(poss), "layers": shape.n_layers,
                   "n_heads": shape.n_heads, "n_kv_heads": shape.n_kv_heads,
                   "head_dim": shape.head_dim, "kv": "q8_0" if shape.kv_q8 else "f32",
                   "step": "layer-serial: per layer one g2b_attn_layers call",
                   "parallelism": "single GPU"},
        "us_per_step": head["us_per_step"],
        "pct_hbm_peak": head["pct_hbm_peak"],
        "bytes_per_step": sb,
        "kv_fill_s": head["kv_fill_s"],
        "roofline": head["roofline"],
        "cpu_baseline": head.get("cpu_baseline"),
        "all_layers_one_call": head.get("all_layers_one_call"),
        "parity_full_size": head.get("parity_full_size"),
        "all_configs": others,
        "gemv": gemv,
        "model_forward": model,
    }
    print(json.dumps(line), flush=True)


def gemv_leg(args):
    """Device weight GEMVs (g2b_matmul, matmul_q of l2_codec.c:342-360) on
    Qwen3-0.6B's output projection (vocab 151936 x dim 1024), the largest
    single matmul_q call of a decode step: weight GB/s of each fused type and
    of F16 / Q4_1 (the reference's dequantising fallback), with the
    reference's own AVX2+OpenMP matmul_q (compiled reference, when it
    was built; else the oracle's scalar restatement on one thread) timed on
    the host cores as the CPU baseline, and a row sample checked against the
    float64 product."""
    from oracle import orc  # CPU baseline and checker only

    n, d = 1024, 151936
    rng = np.random.default_rng(args.seed + 7)
    ctx = attn.Context(attn.Shape(1, 2, 1, 64, 1e4, attn.ARCH_QWEN3, False))
    x = rng.standard_normal(n).astype(np.float32)
    xd = hip.to_device(x)
    od = hip.DeviceBuffer(d * 4)
    res = {"workload": f"Qwen3-0.6B output projection: d={d} rows x n={n}, x ~ N(0,1)",
           "unit": "GB/s of weight bytes"}
    ref = orc.ref_lib("avx2")
    for t, name in ((attn.T_Q8_0, "q8_0"), (attn.T_Q4_0, "q4_0"), (attn.T_F32, "f32"),
                    (attn.T_F16, "f16"), (attn.T_Q4_1, "q4_1")):
        w = orc.random_weights(rng, t, n, d)
        # Launches cycle through copies of the matrix totalling at least
        # GEMV_COLD_BYTES, so that each reads its weights from HBM: a matrix
        # under the 256 MB of MI355X's last-level cache, launched back to
        # back, would otherwise be partly served from that cache.
        ncopy = max(2, -(-GEMV_COLD_BYTES // w.nbytes))
        wds = [ctx.weights_upload(w) for _ in range(ncopy)]
        for k in range(ncopy):
            ctx.matmul(od.ptr, xd.ptr, wds[k], t, n, d)
        ctx.sync()
        e0, e1 = hip.Event(), hip.Event()
        K = ncopy * max(1, -(-max(20, args.steps * 5) // ncopy))
        e0.record(ctx.stream)
        for k in range(K):
            ctx.matmul(od.ptr, xd.ptr, wds[k % ncopy], t, n, d)
        e1.record(ctx.stream)
        e1.synchronize()
        us = e0.elapsed_ms(e1) / K * 1e3
        out = od.download(np.float32, d)
        for wd in wds:
            ctx.weights_free(wd)
        rows = np.sort(rng.choice(d, 4096, replace=False))
        wr = w.reshape(d, -1)[rows].reshape(-1)
        ex, ab = orc.matmul_exact(x, wr, t, n, len(rows))
        rel = float(np.max(np.abs(out[rows] - ex) / ab))
        # CPU baseline: whole matrix, repeated for about a second
        reps, t0 = 0, time.perf_counter()
        while True:
            if ref is not None:
                orc.ref_matmul(x, w, t, n, d, "avx2")
            else:
                orc.matmul_scalar(x, w, t, n, d)
            reps += 1
            if time.perf_counter() - t0 >= 1.0:
                break
        cpu_s = (time.perf_counter() - t0) / reps
        res[name] = {"us": round(us, 2), "GBps": round(w.nbytes / us / 1e3, 1),
                     "copies_cycled": ncopy,
                     "pct_hbm_peak": round(100 * w.nbytes / us / 1e3 / HBM_PEAK_GBPS, 1),
                     "weight_bytes": int(w.nbytes),
                     "max_err_over_sum_abs": rel,
                     "cpu_GBps": round(w.nbytes / cpu_s / 1e9, 2),
                     "cpu_kind": ("reference matmul (AVX2, OpenMP)" if ref is not None
                                  else "oracle scalar restatement, 1 thread"),
                     "cpu_threads": orc.max_threads() if ref is not None else 1}
        log(f"gemv {name}: {us:.1f} us, {res[name]['GBps']} GB/s "
            f"({res[name]['pct_hbm_peak']}% of HBM peak), err/sum|wx| {rel:.1e}, "
            f"cpu {res[name]['cpu_GBps']} GB/s")
    ctx.close()
    return res


def model_leg(args):
    """A whole decode step on the device (g2b_model_forward, model_forward of
    l5_model.c:461-606) for a Qwen3-0.6B-shape model with random Q8_0 weights
    (28 layers, dim 1024, hidden 3072, 16/8 heads of 128, vocab 151936, tied
    embeddings, QK-RMSNorm; 0.63 GB) written as a G2BX file, Q8_0 KV, in two
    windows: positions 8..8+K (below 128: the attention is the single-span
    short kernel) and positions from 4096 (the KV of positions 0..4095
    filled with seeded rows on the device; the attention schedule the
    automatic choice took is recorded).  Beside each, the reference's own
    model_forward (compiled reference, AVX2+OpenMP) on the same file - for
    the long window on the same KV bytes - whose first steps also check the
    device's logits."""
    import tempfile
    from oracle import orc  # CPU baseline and checker only
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from helpers import F_QK_NORM, F_TIE_EMBD, random_model_slots, write_g2bx

    cfg = dict(dim=1024, hidden_dim=3072, n_layers=28, n_heads=16, n_kv_heads=8, vocab=151936,
               seq_len=8192, head_dim=128, eps=1e-6, rope_theta=1e6)
    flags = F_QK_NORM | F_TIE_EMBD
    rng = np.random.default_rng(args.seed + 11)
    P0 = 4096
    fd, path = tempfile.mkstemp(suffix=".g2bx")
    os.close(fd)
    have_ref = orc.ref_lib("avx2") is not None

    def rel_diff(dev, ref):
        return max(float(np.abs(dev[i] - ref[i]).max() / max(1.0, np.abs(ref[i]).max()))
                   for i in range(len(ref)))

    try:
        slots = random_model_slots(rng, cfg, flags, attn.T_Q8_0, attn.T_Q8_0, None)
        wbytes = sum(len(s[3]) for s in slots)
        write_g2bx(path, cfg, attn.ARCH_QWEN3, flags, slots)
        del slots
        K = max(16, args.steps * 2)
        toks = [int(t) for t in rng.integers(0, cfg["vocab"], 8 + K)]
        with attn.Model(path, kv_q8=True) as m:
            first = [m.forward(toks[i], i) for i in range(8)]
            t0 = time.perf_counter()
            for i in range(8, 8 + K):
                m.forward(toks[i], i)
            dt = (time.perf_counter() - t0) / K
            # the long window: positions 0..P0-1 of every layer filled on the
            # device (seeded N(0,1) rows through the append arithmetic)
            kc, vc, cap = m.kv()
            mctx = attn.lib().g2b_model_ctx(m.h)
            rc = attn.lib().g2b_synth_fill_kv(mctx, kc, vc, cap, 0, cfg["n_layers"], 0, P0,
                                              args.seed, 0, float("inf"))
            if rc or attn.lib().g2b_sync(mctx):
                raise RuntimeError(f"KV fill of the model failed ({rc})")
            nbytes = attn.kv_bytes(attn.Shape(cfg["n_layers"], 16, 8, 128, 1e6,
                                              attn.ARCH_QWEN3, True), cap)
            kbytes = hip.copy_d2h(kc, np.uint8, nbytes) if have_ref else None
            vbytes = hip.copy_d2h(vc, np.uint8, nbytes) if have_ref else None
            ltoks = [int(t) for t in rng.integers(0, cfg["vocab"], 4 + K)]
            lfirst = [m.forward(ltoks[i], P0 + i) for i in range(4)]
            t0 = time.perf_counter()
            for i in range(4, 4 + K):
                m.forward(ltoks[i], P0 + i)
            ldt = (time.perf_counter() - t0) / K
            sched = (C.c_int32 * attn.SCHED_FIELDS)()
            attn.lib().g2b_ctx_last_schedule(mctx, sched)
            lsched = attn.schedule_dict(attn.Shape(cfg["n_layers"], 16, 8, 128, 1e6,
                                                   attn.ARCH_QWEN3, True), sched)
            kv_cap = cap
        res = {"workload": "Qwen3-0.6B shape, random Q8_0 weights (tied embeddings, QK-RMSNorm), "
                           "Q8_0 KV, batch 1",
               "weight_bytes": int(wbytes),
               "short_context": {
                   "positions": f"8..{8 + K - 1}", "attention": "k_short, one span",
                   "ms_per_token": round(dt * 1e3, 3), "tokens_per_s": round(1 / dt, 1),
                   "weight_GBps": round(wbytes / dt / 1e9, 1),
                   # embedding, 5 per layer (four fused GEMVs and the attention),
                   # logits
                   "launches_per_token": cfg["n_layers"] * 5 + 2},
               "long_context": {
                   "positions": f"{P0}..{P0 + 3 + K}", "kv_positions_filled": P0,
                   "attention_schedule": lsched,
                   "ms_per_token": round(ldt * 1e3, 3), "tokens_per_s": round(1 / ldt, 1),
                   # plus the combine launch per layer where the splits are not
                   # merged in the decode kernel
                   "launches_per_token": cfg["n_layers"] * (
                       5 if lsched["output_in_kernel"] else 6) + 2}}
        if have_ref:
            # per-token time of the reference: its token loop alone (the driver
            # times it, without the file load and KV allocation), after one
            # untimed call that pages the file in and starts the OpenMP threads
            orc.ref_model_forward(path, toks[:1], cfg["vocab"], True, 0)
            ref_q8, secs = orc.ref_model_forward(path, toks[:8], cfg["vocab"], True, 0,
                                                 timed=True)
            ref_f32 = orc.ref_model_forward(path, toks[:5], cfg["vocab"], False, 0)
            with attn.Model(path, kv_q8=False) as m32:
                dev_f32 = [m32.forward(toks[i], i) for i in range(5)]
            lref, lsecs = orc.ref_model_forward_kv(path, True, kv_cap, kbytes, vbytes, P0,
                                                   ltoks[:4], cfg["vocab"])
            res["short_context"].update({
                "cpu_tokens_per_s": round(8 / secs, 2),
                "max_rel_logit_diff_vs_reference_f32_kv": rel_diff(dev_f32, ref_f32),
                "max_rel_logit_diff_vs_reference_q8_kv": rel_diff(first[:5], ref_q8[:5])})
            res["long_context"].update({
                "cpu_tokens_per_s": round(4 / lsecs, 2),
                "max_rel_logit_diff_vs_reference_q8_kv": rel_diff(lfirst, lref)})
            res.update({"cpu_kind": "reference model_forward (AVX2, OpenMP)",
                        "cpu_threads": orc.max_threads(),
                        "note": "Q8_0 KV: appended rows can quantise one step apart where the "
                                "two fp32 k/v differ in their last bits; the difference compounds "
                                "over 28 layers (argmax unchanged)"})
        log(f"model_forward: {res['short_context']['ms_per_token']} ms/token at positions "
            f"8.., {res['long_context']['ms_per_token']} ms/token at {P0}..; cpu "
            f"{res['short_context'].get('cpu_tokens_per_s')} / "
            f"{res['long_context'].get('cpu_tokens_per_s')} tokens/s")
        return res
    finally:
        os.unlink(path)


def phases_leg(w: Workload, steps: int, warmup: int) -> dict:
    """Where a layer-serial launch's time goes, from the phase-stamp build:
    thread 0 of every workgroup of a k_layer launch reads the device's
    constant wall clock at entry, after the setup (loads, QK-RMSNorm, RoPE,
    digit planes, the owner's append), after the stream of its positions,
    after the fold of its waves' position slots, after the merge and the
    partial stores, and at exit, and notes its XCD (a work-queue workgroup:
    its visits, and the phases of its last one); every combine workgroup at
    entry and exit.  The steps run as the bench runs them (every layer's
    launches back to back; each call writes its own stamp region, read once
    per step).  Per launch: the spread of the workgroups' starts (in all and
    within one XCD), each phase's median over the workgroups, the first
    start to the last exit, and the combine after it; medians over every
    layer call of the timed steps."""
    ctx, s = w.ctx, w.shape
    khz = hip.wall_clock_khz(0)
    cap = max(4096, w.n_seq * 64)
    ctx.stamps_enable(cap, s.n_layers)
    for _ in range(max(1, warmup)):
        w.step_layer_serial()
        ctx.stamps_read()
    rec = []
    for _ in range(steps):
        w.step_layer_serial()
        rec.append((ctx.stamps_read(), ctx.last_schedule()))
    us = 1e3 / khz  # microseconds per tick
    per = collections.defaultdict(list)
    sched = rec[0][1]
    wq = sched.get("piece_len", 0) > 0
    for st_all, sc in rec:
        prev_end = None
        for st in st_all:
            ks = st[0][st[0][:, 5] != 0].astype(np.int64)
            cs = st[1][st[1][:, 5] != 0].astype(np.int64)
            if len(ks) == 0:
                raise RuntimeError(f"no k_layer stamps (phases need k_layer launches): {sc}")
            t0, t_end = ks[:, 0].min(), ks[:, 5].max()
            per["workgroups"].append(len(ks))
            per["start_spread"].append((ks[:, 0].max() - t0) * us)
            if wq:
                # work queue: the workgroups' exits, visits, and the phases of
                # each workgroup's last visit (its first when it made one)
                ex = (ks[:, 5] - t0) * us
                for q in (10, 50, 90):
                    per[f"exit_p{q}"].append(float(np.percentile(ex, q)))
                per["exit_last"].append(float(ex.max()))
                per["visits_mean"].append(float(ks[:, 6].mean()))
                one = ks[ks[:, 6] == 1]
                if len(one):
                    per["single_visit_setup_from_entry"].append(
                        float(np.median(one[:, 1] - one[:, 0])) * us)
            for name, (a, b) in (("setup", (0, 1)), ("stream", (1, 2)), ("fold", (2, 3)),
                                 ("merge_and_partial_stores", (3, 4)), ("exit", (4, 5)),
                                 ("workgroup_total", (0, 5))):
                if wq and name in ("setup", "workgroup_total"):
                    continue  # (from entry: the last visit's setup follows earlier visits)
                per[name].append(float(np.median(ks[:, b] - ks[:, a])) * us)
            per["first_start_to_last_exit"].append((t_end - t0) * us)
            xcd = ks[:, 7]
            firsts = {int(x): ks[xcd == x, 0].min() for x in np.unique(xcd)}
            per["xcds"].append(len(firsts))
            per["xcd_first_start_spread"].append((max(firsts.values()) - t0) * us)
            per["start_spread_within_xcd"].append(float(np.max(
                [(ks[xcd == x, 0].max() - ks[xcd == x, 0].min()) * us for x in firsts])))
            for x, f in firsts.items():
                per[f"xcd{x}_first_start"].append((f - t0) * us)
            if prev_end is not None:
                per["previous_combine_exit_to_first_start"].append((t0 - prev_end) * us)
            prev_end = t_end
            if len(cs):
                per["gap_to_combine"].append((cs[:, 0].min() - t_end) * us)
                per["combine_first_start_to_last_exit"].append(
                    (cs[:, 5].max() - cs[:, 0].min()) * us)
                per["first_start_to_combine_exit"].append((cs[:, 5].max() - t0) * us)
                prev_end = cs[:, 5].max()
    out = {"workload": w.name, "variant": sched.get("variant"), "schedule": sched,
           "launches": sum(len(r[0]) for r in rec), "wall_clock_khz": khz,
           "unit": "us (medians over the launches; per launch, phase = median over workgroups)"}
    for k, v in sorted(per.items()):
        out[k] = round(float(np.median(v)), 2)
    ev_ms, _, ev_dec, ev_n = w.timed(w.step_layer_serial, steps, warmup)
    out["same_build_events"] = {"layer_serial_us_per_step": round(ev_ms * 1e3, 1),
                                "decode_avg_us": round(ev_dec / max(ev_n, 1) * 1e3, 2)}
    log(f"{w.name} phases: " + ", ".join(f"{k} {out[k]}" for k in sorted(per)))
    return out


def cpu_leg(w: Workload, na: int, nb: int, min_s: float):
    """The CPU baseline and the full-size parity sample of one config: the
    oracle (a C99 restatement of the reference path, built with the
    reference's flags) on the first nb sequences x every layer, with the KV
    bytes and inputs the GPU used, in mode A (the first na sequences in turn
    on one thread, as the reference's single-threaded attention runs them)
    and mode B (OpenMP over the nb sequences, all host threads), each
    repeated for at least min_s seconds.  Its outputs are compared with the
    GPU's layer-serial outputs, the appended rows byte for byte, and up to
    three (sequence, layer) units are also evaluated in float64 from the
    same bytes."""
    from oracle import orc  # CPU baseline and checker only
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from helpers import exact_attention  # float64 checker

    shape, poss, caps, kvs = w.shape, w.poss, w.caps, w.kvs
    o = orc.Shape(shape.n_layers, shape.n_heads, shape.n_kv_heads, shape.head_dim,
                  shape.rope_theta, shape.arch, shape.kv_q8)
    L, nq, nkv, rb = shape.n_layers, shape.nq, shape.nkv, row_bytes(shape)
    n_seq = len(poss)
    nb = max(1, min(nb, n_seq))
    na = max(1, min(na, nb))
    idx = list(range(nb))
    nQ, nK = L * n_seq * nq, L * n_seq * nkv
    q_all = w.q0.download(np.float32, nQ).reshape(L, n_seq, nq)
    k_all = w.kb.download(np.float32, nK).reshape(L, n_seq, nkv)
    v_all = w.vb.download(np.float32, nK).reshape(L, n_seq, nkv)
    out_gpu = w.qw.download(np.float32, nQ).reshape(L, n_seq, nq)
    t0 = time.perf_counter()
    host = []
    for i in idx:
        nbytes = attn.kv_bytes(shape, caps[i])
        host.append((hip.copy_d2h(kvs[i][0], np.uint8, nbytes),
                     hip.copy_d2h(kvs[i][1], np.uint8, nbytes)))
    log(f"{w.name} cpu sample: {nb} sequences copied to host in {time.perf_counter() - t0:.1f}s")
    gpu_rows = [(kc.reshape(L, caps[i], rb)[:, poss[i]].copy(),
                 vc.reshape(L, caps[i], rb)[:, poss[i]].copy()) for i, (kc, vc) in zip(idx, host)]

    def sample(ids, threads):
        """Run the sample repeatedly for at least min_s; seconds per pass."""
        pos = np.array([poss[i] for i in ids], np.int32)
        cap = np.array([caps[i] for i in ids], np.int32)
        sel = np.array(ids)
        q = np.ascontiguousarray(q_all[:, sel])
        k = np.ascontiguousarray(k_all[:, sel])
        v = np.ascontiguousarray(v_all[:, sel])
        reps, t = 0, orc.now()
        while True:
            # (the appended rows are rewritten with the same bytes every pass)
            out = orc.attn_batch(o, 0, L, pos, cap, [host[j][0] for j in range(len(ids))],
                                 [host[j][1] for j in range(len(ids))], q, k, v, threads)
            reps += 1
            if orc.now() - t >= min_s:
                break
        return (orc.now() - t) / reps, out, reps

    threads = orc.max_threads() if nb > 1 else 1
    ta, out_a, reps_a = sample(idx[:na], 1)
    tb, out_b, reps_b = sample(idx, threads)
    bytes_a = step_bytes(shape, [poss[i] for i in idx[:na]])
    bytes_b = step_bytes(shape, [poss[i] for i in idx])
    gbps_a, gbps_b = bytes_a / ta / 1e9, bytes_b / tb / 1e9
    log(f"{w.name} cpu: 1 thread {gbps_a:.2f} GB/s ({reps_a} x {ta:.3f}s), {threads} threads "
        f"{gbps_b:.2f} GB/s ({reps_b} x {tb:.3f}s)")

    err = float(np.max(np.abs(out_b - out_gpu[:, idx])))
    rows_exact = all(
        np.array_equal(host[j][0].reshape(L, caps[i], rb)[:, poss[i]], gpu_rows[j][0]) and
        np.array_equal(host[j][1].reshape(L, caps[i], rb)[:, poss[i]], gpu_rows[j][1])
        for j, i in enumerate(idx))
    # float64 evaluation from the same cache bytes of three units: the first
    # and last sampled sequence (first and last layer) and the unit where the
    # GPU and the oracle differ most.  The tests' rule (helpers.check_out):
    # max |gpu - float64| <= 1e-4, and max |gpu - oracle| <= 1e-4 plus the
    # oracle's own error from float64 (its serial fp32 sums drift at 16k-32k
    # positions), unit by unit.
    per_unit = np.max(np.abs(out_b - out_gpu[:, idx]), axis=2)  # [layer][sample]
    worst_l, worst_j = (int(v) for v in np.unravel_index(np.argmax(per_unit), per_unit.shape))
    f64_gpu = f64_orc = 0.0
    within = True
    units = [(0, 0), (len(idx) - 1, L - 1), (worst_j, worst_l)]
    for j, layer in dict.fromkeys(units):
        i = idx[j]
        ex, _ = exact_attention(o, caps[i], layer, poss[i], host[j][0], host[j][1],
                                q_all[layer, i])
        e_ex = float(np.max(np.abs(out_gpu[layer, i] - ex)))
        own = float(np.max(np.abs(out_b[layer, j] - ex)))
        f64_gpu, f64_orc = max(f64_gpu, e_ex), max(f64_orc, own)
        within &= e_ex <= 1e-4 and float(per_unit[layer, j]) <= 1e-4 + own
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    mode_b = ("OpenMP over sequences, all host threads" if threads > 1 else
              "one sequence: the reference attention has no threads inside a sequence")
    cpu = {"value": round(gbps_b, 3), "unit": "GB/s", "cores": threads, "kind": "port",
           "sample": f"{nb} of {n_seq} sequences x {L} layers ({mode_b}), same KV bytes and "
                     f"inputs as the GPU, {reps_b} passes",
           "us_per_step_of_sample": round(tb * 1e6, 1),
           "seconds": round(tb * reps_b, 2), "cpu": cpu_model,
           "one_thread": {"value": round(gbps_a, 3), "unit": "GB/s", "cores": 1,
                          "sample": f"{na} sequences x {L} layers, sequences in turn "
                                    f"(the reference attention is single-threaded), "
                                    f"{reps_a} passes",
                          "us_per_step_of_sample": round(ta * 1e6, 1),
                          "seconds": round(ta * reps_a, 2)}}
    parity = {"units_checked": nb * L, "max_abs_out_err_vs_oracle": err,
              "appended_rows_bit_exact": bool(rows_exact),
              "float64_units": len(dict.fromkeys(units)),
              "max_abs_out_err_gpu_vs_float64": f64_gpu,
              "max_abs_out_err_oracle_vs_float64": f64_orc,
              "rule": "per unit: |gpu - float64| <= 1e-4 and |gpu - oracle| <= 1e-4 + "
                      "|oracle - float64| (float64 on the first, last and worst unit)",
              "within_rule": bool(within)}
    log(f"{w.name} parity: {nb * L} units, max |gpu - oracle| {err:.3g}, rows bit-exact "
        f"{rows_exact}, float64: gpu {f64_gpu:.3g}, oracle {f64_orc:.3g}, within the rule "
        f"{within}")
    return cpu, parity


if __name__ == "__main__":
    main()
