# -*- coding: utf-8 -*-
"""Benchmark: RVC v2 40k synthesis throughput on one MI355X.

Default workload ("config 2"): full synthesizer
enc_p + flow + GeneratorNSF, fp32, random-init weights, 10 s of 40 kHz audio
(P = 1000 frames), batch 1.  One step = one ``rvc_synth_infer_dev`` call over
inputs already resident in HBM (phone [1,1000,768], pitch, nsff0, sid, the
z_p noise nz and the NSF noise ns), ending with a stream synchronize.

Prints ONE JSON line with the metric, the roofline of the dominant kernel
(the fp32 MFMA implicit-GEMM ResBlock convolutions, timed with HIP events on
the session stream over the timed steps) and a CPU baseline (the numpy
oracle on a bounded 4 s sample of the same workload, on this host).  The
host-in / host-out rate (numpy arrays in, numpy waveform out, PCIe copies
included; the median of 20 calls after 3 warm-ups) is reported beside it as
``host_io_audio_s_per_s``; ``value`` is the device-resident rate.

``--workload hubert`` measures BASELINE config 3 instead (HuBERT-base
encoder, 10 s of 16 kHz audio -> [1, 499, 768]), ``--workload dec48k-b8``
config 4 (48k GeneratorNSF, 8 chunks of 6 s as one batch), ``--workload
synth40k-bf16-b4`` config 5, and ``--workload vc40k`` the device-resident
conversion chain around config 2 (HuBERT, retrieval, synthesis, RMS mix,
int16), and ``--workload rmvpe10s`` RMVPE pitch extraction of 10 s at
16 kHz; each prints its own JSON line in the same format.  The default run
is config 2.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "rvc-vulkan_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

METRIC = "audio-sec synthesized/sec (10 s @40 kHz, 1 GPU) + HBM GB/s & MFMA util per op"
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0  # dense bf16 MFMA
SR = 40000
P_FRAMES = 1000           # 10 s at 100 frames/s
CPU_SAMPLE_FRAMES = 400   # 4 s sample for the numpy baseline (about 10 s of CPU work)


def _log(msg):
    print(msg, file=sys.stderr, flush=True)


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "synth_40k_resblock_traffic.md")


def family_entry(t, peak_tflops=PEAK_FP32_TFLOPS):
    """ms, TFLOP/s, GB/s of one timing family, and its roofline fraction
    achieved / min(peak FLOP/s, AI x peak HBM bandwidth), AI = FLOPs / bytes."""
    ms, fl, by = t["ms"], t["flops"], t["bytes"]
    e = {"ms": round(ms, 4), "tflops": None, "gbs": None, "roof_frac": None}
    if ms > 0:
        tf = fl / (ms / 1e3) / 1e12
        gbs = by / (ms / 1e3) / 1e9
        e["tflops"], e["gbs"] = round(tf, 2), round(gbs, 1)
        roof_tf = min(peak_tflops, (fl / by) * PEAK_HBM_GBS / 1e3) if by > 0 and fl > 0 else None
        if roof_tf:
            e["roof_frac"] = round(tf / roof_tf, 3)
        elif by > 0:
            e["roof_frac"] = round(gbs / PEAK_HBM_GBS, 3)
    return e


def profiled_traffic():
    """HBM bytes per ResBlock launch from the committed PMC summary (FETCH_SIZE
    and WRITE_SIZE runs of this benchmark, copy-calibrated; written by
    ``python -m rvc_hip.profsum --traffic``), or None when it is absent."""
    import re

    try:
        with open(TRAFFIC_PROFILE) as f:
            m = re.search(r"resblock_traffic_bytes_per_launch: (\d+)", f.read())
    except OSError:
        return None
    return int(m.group(1)) if m else None


def host_cpu():
    """Model name, physical cores and logical threads of this host (from
    /proc/cpuinfo, which is what lscpu reads)."""
    model, cores = "unknown", set()
    try:
        phys = core = None
        with open("/proc/cpuinfo") as f:
            for ln in f:
                k, _, v = ln.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model == "unknown":
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None:
                    cores.add((phys, core))
                    phys = core = None
            if phys is not None:
                cores.add((phys, core))
    except OSError:
        pass
    return {"model": model, "physical_cores": len(cores) or None, "threads": os.cpu_count()}


def cpu_baseline(w, geom):
    """The numpy oracle (a restatement of the reference numpy path) on a 4 s
    sample of the same workload; returns audio-seconds per second."""
    from oracle import vits_ref
    from rvc_hip import synthetic as syn

    threads = _blas_threads()
    ref = vits_ref.Synthesizer(w, sr=geom.sr)
    inp = syn.make_synth_inputs(geom, CPU_SAMPLE_FRAMES, seed=7)
    ref.infer_controlled(inp["phone"][:, :10], inp["pitch"][:, :10], inp["nsff0"][:, :10], inp["sid"],
                         inp["nz"][:, :, :10], inp["ns"][:, :10 * geom.upp])  # warm BLAS / allocator
    t0 = time.perf_counter()
    ref.infer_controlled(inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"], inp["nz"], inp["ns"])
    dt = time.perf_counter() - t0
    audio_s = CPU_SAMPLE_FRAMES / 100.0
    return {"value": audio_s / dt, "unit": "audio-s/s", "cores": int(threads), "kind": "port",
            "sample": f"{CPU_SAMPLE_FRAMES / 100:g} s (P={CPU_SAMPLE_FRAMES}) of the config-2 synthesis (same weights, 40k), "
                      f"numpy oracle, 1 run after a warm-up, {dt:.2f} s wall",
            "host": host_cpu(), "blas_threads": int(threads)}


def calibrate_copy(mib: int):
    """rvc_copy of ``mib`` MiB, 5 launches: each reads and writes exactly
    ``mib`` MiB, so FETCH_SIZE / WRITE_SIZE per dispatch should read
    ``mib * 1024`` KiB; the ratio scales the counters of the other kernels."""
    from rvc_hip import _hip
    from rvc_hip.hip_ops import get_context

    ctx = get_context()
    n = mib * (1 << 20) // 4
    src = ctx.upload(np.random.default_rng(0).standard_normal(n).astype(np.float32))
    dst = ctx.alloc(n)
    lib = _hip.get_lib()
    for _ in range(5):
        _hip._check(lib.rvc_copy(ctx.handle, dst, src, n), "rvc_copy")
    ctx.download(dst, (4,))
    print(json.dumps({"copy_bytes_per_launch": n * 4, "launches": 5}), flush=True)
    return 0


def bench_hubert(args):
    """HuBERT-base, 160 000 samples at 16 kHz, batch 1."""
    from rvc_hip import _hip, synthetic as syn
    from rvc_hip.hip_ops import get_context
    from rvc_hip.hubert import HipHubert

    T = 160000
    sd = syn.make_hubert_weights(syn.HUBERT_BASE, seed=0)
    ctx = get_context()
    hub = HipHubert(sd, ctx=ctx)
    _log(f"bench: device {_hip.device_name()}; HuBERT weights resident")
    x = syn.make_hubert_input(T, seed=3)
    L = hub.frames(T)
    xid = ctx.upload(x)
    oid = ctx.alloc(L * 768)

    def step():
        hub.encode_dev(xid, 1, T, oid, version=2)

    for _ in range(args.warmup):
        step()
    hub.set_timing("hub.ffn")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    dt = time.perf_counter() - t0
    fam = hub.get_timing()
    hub.set_timing("")
    breakdown = {}
    for tag in () if args.quick else ("hub.conv0", "hub.gn", "hub.conv", "hub.proj", "hub.pos", "hub.qkv", "hub.attn",
                                      "hub.o", "hub.ln", "hub.ffn"):
        hub.set_timing(tag)
        step()
        t = hub.get_timing()
        breakdown[tag] = {"ms": round(t["ms"], 4),
                          "tflops": round(t["flops"] / (t["ms"] / 1e3) / 1e12, 2) if t["ms"] > 0 else None,
                          "gbs": round(t["bytes"] / (t["ms"] / 1e3) / 1e9, 1) if t["ms"] > 0 else None}
    hub.set_timing("")
    audio_s = T / 16000.0
    value = audio_s * args.steps / dt
    n = max(fam["launches"], 1)
    avg_s = fam["ms"] / 1e3 / n
    achieved = fam["flops"] / n / avg_s / 1e12 if avg_s > 0 else 0.0
    # the FFN family: per layer the input GEMM and the output GEMM's two
    # C_in halves plus their ordered reduce (three launches)
    roofline = {"kernel": "conv_small (HuBERT FFN 1x1 GEMMs 768->3072->768, output GEMM split-K + reduce)",
                "bound": "mfma",
                "achieved": round(achieved, 2), "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_FP32_TFLOPS, 4), "traffic": None,
                "avg_launch_us": round(avg_s * 1e6, 2), "launches_per_step": n // args.steps,
                "share_of_step": round(fam["ms"] / (dt * 1e3), 3)}
    cpu = None
    if not (args.no_cpu_baseline or args.quick):
        from oracle import hubert_ref

        ref = hubert_ref.HubertRef(sd)
        xs = syn.make_hubert_input(16000, seed=7)
        ref.encode(xs[:, :4000])
        t0 = time.perf_counter()
        ref.encode(xs)
        cdt = time.perf_counter() - t0
        cpu = {"value": 1.0 / cdt, "unit": "audio-s/s", "cores": _blas_threads(), "kind": "port",
               "sample": f"1 s (16 000 samples) of the config-3 encode (same weights), numpy oracle, 1 run after "
                         f"a warm-up, {cdt:.2f} s wall"}
    line = {
        "metric": "audio-sec encoded/sec (HuBERT-base, 10 s @16 kHz, 1 GPU)", "value": round(value, 2),
        "unit": "audio-s/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded input, random-init weights)",
        "config": {"workload": "config 3: HuBERT-base encoder, 160000 samples @16 kHz -> [1,499,768], batch 1, fp32",
                   "samples": T, "frames": L, "batch": 1},
        "roofline": roofline, "cpu_baseline": cpu, "breakdown": breakdown,
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_dec48(args):
    """48k GeneratorNSF, 8 chunks of 6 s (P=600) as one batch."""
    from rvc_hip import _hip, synthetic as syn
    from rvc_hip.hip_ops import get_context
    from rvc_hip.synth import HipSynthesizer

    geom = syn.GEOM_48K
    w = syn.make_weights(geom, seed=0)
    ctx = get_context()
    s = HipSynthesizer(w, sr=geom.sr, ctx=ctx)
    _log(f"bench: device {_hip.device_name()}; 48k weights resident")
    B, P = 8, 600
    ins = [syn.make_dec_inputs(geom, P, seed=60 + i) for i in range(B)]
    z = np.concatenate([i["z"] for i in ins]).astype(np.float32)
    f0 = np.concatenate([i["f0"] for i in ins]).astype(np.float32)
    g = np.repeat(ins[0]["g"].reshape(1, -1), B, axis=0).astype(np.float32)
    ns = np.concatenate([i["ns"].reshape(1, -1) for i in ins]).astype(np.float32)
    ids = [ctx.upload(np.ascontiguousarray(a)) for a in (z, f0, g, ns)]
    wave = ctx.alloc(B * P * geom.upp)

    def step():
        s.decode_dev(ids[0], ids[1], ids[2], ids[3], B, P, wave)

    for _ in range(args.warmup):
        step()
    s.set_timing("dec.rb")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    dt = time.perf_counter() - t0
    rb = s.get_timing()
    s.set_timing("")
    audio_s = B * P / 100.0
    value = audio_s * args.steps / dt
    n = max(rb["launches"], 1)
    avg_s = rb["ms"] / 1e3 / n
    achieved = rb["flops"] / n / avg_s / 1e12 if avg_s > 0 else 0.0
    roofline = {"kernel": "conv1d_mfma (GeneratorNSF ResBlock convs, all stages)", "bound": "mfma",
                "achieved": round(achieved, 2), "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_FP32_TFLOPS, 4), "traffic": None,
                "avg_launch_us": round(avg_s * 1e6, 2), "launches_per_step": n // args.steps,
                "share_of_step": round(rb["ms"] / (dt * 1e3), 3)}
    cpu = None
    if not (args.no_cpu_baseline or args.quick):
        from oracle import vits_ref

        dec = vits_ref.GeneratorNSF(w, vits_ref.VitsConfig(w, sr=geom.sr))
        d = syn.make_dec_inputs(geom, 100, seed=9)
        dec.forward(d["z"][:, :, :10], d["f0"][:, :10], d["g"], d["ns"][:, :10 * geom.upp])
        t0 = time.perf_counter()
        dec.forward(d["z"], d["f0"], d["g"], d["ns"])
        cdt = time.perf_counter() - t0
        cpu = {"value": 1.0 / cdt, "unit": "audio-s/s", "cores": _blas_threads(), "kind": "port",
               "sample": f"1 s (P=100) of one config-4 chunk (same 48k weights), numpy oracle, 1 run after a "
                         f"warm-up, {cdt:.2f} s wall"}
    line = {
        "metric": "audio-sec synthesized/sec (48k GeneratorNSF, 8 x 6 s chunks as batch 8, 1 GPU)",
        "value": round(value, 2), "unit": "audio-s/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded inputs, random-init weights)",
        "config": {"workload": "config 4: RVC v2 48k GeneratorNSF, 8 chunks x P=600 (6 s) as batch 8, fp32",
                   "frames": P, "batch": B, "sample_rate": geom.sr, "chunk_audio_s_per_step": audio_s},
        "roofline": roofline, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def _blas_threads():
    try:
        from threadpoolctl import threadpool_info

        return int(max((i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"),
                       default=1))
    except Exception:  # noqa: BLE001
        return 1


def bench_bf16(args, precision):
    """config 2 x 4 independent seeds as one batch of 4, with
    the GeneratorNSF upsample ConvTranspose1d and the enc_p matmuls on bf16
    MFMA, fp32 accumulate (precision 1); precision 2 also puts the decoder
    ResBlocks on bf16 (reported separately).  The waveform SNR against the
    fp32 path on the same inputs is measured in the same run (untimed)."""
    import math

    from rvc_hip import _hip, synthetic as syn
    from rvc_hip.hip_ops import get_context
    from rvc_hip.synth import HipSynthesizer

    if not _hip.has_so:
        raise RuntimeError(f"HIP backend missing: {_hip.so_load_error}")
    geom = syn.GEOM_40K
    w = syn.make_weights(geom, seed=0)
    ctx = get_context()
    s = HipSynthesizer(w, sr=geom.sr, ctx=ctx, precision=precision)
    P, B = P_FRAMES, 4
    ins = [syn.make_synth_inputs(geom, P, seed=sd) for sd in (41, 42, 43, 44)]
    cat = {k: np.ascontiguousarray(np.concatenate([i[k] for i in ins], axis=0)) for k in
           ("phone", "pitch", "nsff0", "sid", "nz", "ns")}
    ids = {
        "phone": ctx.upload(cat["phone"].astype(np.float32)),
        "pitch": ctx.upload(cat["pitch"].astype(np.int64)),
        "f0": ctx.upload(cat["nsff0"].astype(np.float32)),
        "sid": ctx.upload(cat["sid"].astype(np.int64)),
        "nz": ctx.upload(cat["nz"].astype(np.float32)),
        "ns": ctx.upload(cat["ns"].astype(np.float32).reshape(-1)),
    }
    n_out = P * geom.upp
    wave_id = ctx.alloc(B * n_out)

    def step():
        s.infer_dev(ids["phone"], ids["pitch"], ids["f0"], ids["sid"], ids["nz"], ids["ns"], B, P, wave_id)

    for _ in range(args.warmup):
        step()
    s.set_timing("dec.rb")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    dt = time.perf_counter() - t0
    rb = s.get_timing()
    s.set_timing("")
    ms_step = dt * 1e3 / args.steps
    audio_s = P / 100.0 * B
    value = audio_s * args.steps / dt
    _log(f"bench config 5 (precision {precision}): {ms_step:.3f} ms/step, {value:.1f} audio-s/s")
    y = ctx.download(wave_id, (B, 1, n_out))

    peak_rb = PEAK_BF16_TFLOPS if precision >= 2 else PEAK_FP32_TFLOPS
    n_launch = max(rb["launches"], 1)
    avg_s = rb["ms"] / 1e3 / n_launch
    achieved = rb["flops"] / n_launch / avg_s / 1e12 if avg_s > 0 else 0.0
    roofline = {"kernel": "conv1d_" + ("bf16" if precision >= 2 else "mfma") + " (GeneratorNSF ResBlock convs)",
                "bound": "mfma", "achieved": round(achieved, 2), "peak": peak_rb, "unit": "TFLOP/s",
                "frac": round(achieved / peak_rb, 4), "traffic": None,
                "avg_launch_us": round(avg_s * 1e6, 2), "launches_per_step": n_launch // args.steps,
                "share_of_step": round(rb["ms"] / (dt * 1e3), 3)}
    breakdown = {}
    for tag, peak in (("dec.rb", peak_rb), ("dec.ups", PEAK_BF16_TFLOPS), ("enc", PEAK_BF16_TFLOPS),
                      ("flow", PEAK_FP32_TFLOPS)):
        if args.quick:
            break
        s.set_timing(tag)
        step()
        breakdown[tag] = family_entry(s.get_timing(), peak)
    s.set_timing("")
    snr = None
    if not args.quick:
        ref = HipSynthesizer(w, sr=geom.sr, ctx=ctx, precision=0)
        y0 = ref.infer_controlled(cat["phone"], cat["pitch"], cat["nsff0"], cat["sid"], cat["nz"], cat["ns"])
        ref.close()
        snr = min(10.0 * math.log10(float((y0[b].astype(np.float64) ** 2).sum()) /
                                    max(float(((y[b].astype(np.float64) - y0[b]) ** 2).sum()), 1e-300))
                  for b in range(B))
    what = "ups + enc_p matmuls" if precision == 1 else "ups + enc_p matmuls + ResBlocks"
    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "audio-s/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 (" + what + "), f32 elsewhere; f32 accumulate",
        "data": "synthetic (4 seeded inputs, random-init weights)",
        "config": {"workload": f"config 5: config 2 x 4 seeds as batch 4, {what} on bf16 MFMA",
                   "frames": P, "batch": B, "sample_rate": SR, "output_samples": n_out},
        "roofline": roofline, "cpu_baseline": None,
        "snr_db_vs_fp32": None if snr is None else round(snr, 2), "snr_bar_db": 40.0,
        "breakdown": breakdown,
    }
    print(json.dumps(line), flush=True)
    return 0


VC_INDEX_ROWS = 20000  # retrieval index size of the vc40k workload (HuBERT-v2 width 768)


def bench_vc(args):
    """The device-resident conversion chain around config 2 (not a BASELINE
    config; reported beside it): 10 s of 16 kHz input -> HuBERT-base
    (config 3) -> retrieval blend against a 20 000-row index at index_rate
    0.75, 2x interpolation and the protect mask (protect 0.33) -> the 40k
    synthesizer of config 2 on the 2 x 499 = 998 frames -> change_rms
    (rate 0.25) -> int16.  Pitch is an input (F0 extraction is outside this
    backend).  One step = the five device calls on resident buffers."""
    from rvc_hip import _hip, synthetic as syn
    from rvc_hip.hip_ops import get_context
    from rvc_hip.hubert import HipHubert
    from rvc_hip.pipeline import HipVcGlue
    from rvc_hip.synth import HipSynthesizer

    if not _hip.has_so:
        raise RuntimeError(f"HIP backend missing: {_hip.so_load_error}")
    ctx = get_context()
    geom = syn.GEOM_40K
    T = 160000
    hub = HipHubert(syn.make_hubert_weights(syn.HUBERT_BASE, seed=0), ctx=ctx)
    s = HipSynthesizer(syn.make_weights(geom, seed=0), sr=geom.sr, ctx=ctx)
    glue = HipVcGlue(ctx)
    rng = np.random.default_rng(5)
    glue.set_index(rng.standard_normal((VC_INDEX_ROWS, 768)).astype(np.float32))
    _log(f"bench: device {_hip.device_name()}; HuBERT, synthesizer and index resident")
    L = hub.frames(T)
    P = 2 * L
    inp = syn.make_synth_inputs(geom, P, seed=3)
    x = syn.make_hubert_input(T, seed=3)
    ids = {
        "x": ctx.upload(x), "feats": ctx.alloc(L * 768), "phone": ctx.alloc(P * 768),
        "pitch": ctx.upload(np.ascontiguousarray(inp["pitch"], np.int64)),
        "f0": ctx.upload(np.ascontiguousarray(inp["nsff0"], np.float32)),
        "sid": ctx.upload(np.ascontiguousarray(inp["sid"], np.int64)),
        "nz": ctx.upload(np.ascontiguousarray(inp["nz"], np.float32)),
        "ns": ctx.upload(np.ascontiguousarray(inp["ns"], np.float32).reshape(-1)),
    }
    n_out = P * geom.upp
    ids["wave"] = ctx.alloc(n_out)
    ids["mix"] = ctx.alloc(n_out)
    ids["i16"] = ctx.alloc((n_out + 1) // 2)
    stages = {
        "hubert": lambda: hub.encode_dev(ids["x"], 1, T, ids["feats"], version=2),
        "prepare": lambda: glue.prepare_dev(ids["feats"], L, 768, 0.75, ids["f0"], 0.33, ids["phone"]),
        "synth": lambda: s.infer_dev(ids["phone"], ids["pitch"], ids["f0"], ids["sid"], ids["nz"], ids["ns"], 1, P,
                                     ids["wave"]),
        "change_rms": lambda: glue.change_rms_dev(ids["x"], T, 16000, ids["wave"], n_out, geom.sr, 0.25, ids["mix"]),
        "int16": lambda: _hip._check(_hip.get_lib().rvc_vc_to_int16_dev(glue.handle, ids["mix"], n_out, ids["i16"]),
                                     "rvc_vc_to_int16_dev"),
    }

    def step():
        for fn in stages.values():
            fn()

    for _ in range(args.warmup):
        step()
    s.set_timing("dec.rb")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    dt = time.perf_counter() - t0
    rb = s.get_timing()
    s.set_timing("")
    audio_s = T / 16000.0
    value = audio_s * args.steps / dt
    _log(f"bench vc40k: {dt * 1e3 / args.steps:.3f} ms/step, {value:.1f} audio-s/s")
    n = max(rb["launches"], 1)
    avg_s = rb["ms"] / 1e3 / n
    achieved = rb["flops"] / n / avg_s / 1e12 if avg_s > 0 else 0.0
    roofline = {"kernel": "conv1d_mfma (GeneratorNSF ResBlock convs, all stages)", "bound": "mfma",
                "achieved": round(achieved, 2), "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_FP32_TFLOPS, 4), "traffic": None,
                "avg_launch_us": round(avg_s * 1e6, 2), "launches_per_step": n // args.steps,
                "share_of_step": round(rb["ms"] / (dt * 1e3), 3)}
    breakdown = {}
    if not args.quick:
        reps = 5
        for name, fn in stages.items():
            t0 = time.perf_counter()
            for _ in range(reps):
                fn()
            breakdown[name] = {"ms": round((time.perf_counter() - t0) * 1e3 / reps, 4)}
        for tag in ("vc.knn.gemm", "vc.knn.select", "vc.blend", "vc.interp", "vc.rms", "vc.int16"):
            glue.set_timing(tag)
            stages["prepare"]()
            stages["change_rms"]()
            stages["int16"]()
            breakdown[tag] = family_entry(glue.get_timing())
        glue.set_timing("")
    line = {
        "metric": "audio-sec converted/sec (HuBERT + retrieval + 40k synthesis + RMS mix, 10 s @16 kHz in, 1 GPU)",
        "value": round(value, 2), "unit": "audio-s/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded input, random-init weights and index)",
        "config": {"workload": f"vc40k: 160000 samples @16 kHz -> HuBERT-base [1,{L},768] -> retrieval over "
                               f"{VC_INDEX_ROWS} rows (index_rate 0.75) + 2x interpolation + protect 0.33 -> "
                               f"40k synthesis P={P} -> change_rms 0.25 -> int16",
                   "samples_in": T, "frames": P, "batch": 1, "index_rows": VC_INDEX_ROWS, "output_samples": n_out},
        "roofline": roofline, "cpu_baseline": None, "breakdown": breakdown,
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_rmvpe(args):
    """RMVPE f0 extraction (the pipeline's pitch model), 160 000 samples at
    16 kHz -> f0 [1001], batch 1, fp32, device-resident."""
    from rvc_hip import _hip, synthetic as syn
    from rvc_hip.hip_ops import get_context
    from rvc_hip.rmvpe import HipRMVPE

    T = 160000
    w = syn.make_rmvpe_weights(seed=0)
    ctx = get_context()
    m = HipRMVPE(w, ctx=ctx)
    _log(f"bench: device {_hip.device_name()}; RMVPE weights resident")
    x = syn.make_rmvpe_audio(T, seed=5)
    F = m.frames(T)
    xid = ctx.upload(x)
    fid = ctx.alloc(F)

    def step():
        m.infer_dev(xid, T, fid)

    for _ in range(args.warmup):
        step()
    m.set_timing("rmvpe.enc")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    dt = time.perf_counter() - t0
    fam = m.timing()
    m.set_timing("")
    breakdown = {}
    for tag in () if args.quick else ("rmvpe.mel", "rmvpe.enc", "rmvpe.pool", "rmvpe.inter", "rmvpe.dec",
                                      "rmvpe.head", "rmvpe.gru", "rmvpe.decode"):
        m.set_timing(tag)
        step()
        t = m.timing()
        breakdown[tag] = {"ms": round(t["ms"], 4), "launches": t["launches"],
                          "tflops": round(t["flops"] / (t["ms"] / 1e3) / 1e12, 2) if t["ms"] > 0 else None}
    m.set_timing("")
    audio_s = T / 16000.0
    value = audio_s * args.steps / dt
    n = max(fam["launches"], 1)
    avg_s = fam["ms"] / 1e3 / n
    achieved = fam["flops"] / n / avg_s / 1e12 if avg_s > 0 else 0.0
    roofline = {"kernel": "conv2d_mfma (RMVPE encoder ConvBlockRes 3x3 convs)", "bound": "mfma",
                "achieved": round(achieved, 2), "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_FP32_TFLOPS, 4), "traffic": None,
                "avg_launch_us": round(avg_s * 1e6, 2), "launches_per_step": n // args.steps,
                "share_of_step": round(fam["ms"] / (dt * 1e3), 3)}
    cpu = None
    if not (args.no_cpu_baseline or args.quick):
        from oracle import rmvpe_ref

        ref = rmvpe_ref.Rmvpe(w)
        xs = syn.make_rmvpe_audio(16000, seed=7)
        ref.infer_from_audio(xs[:4000])
        t0 = time.perf_counter()
        ref.infer_from_audio(xs)
        cdt = time.perf_counter() - t0
        cpu = {"value": 1.0 / cdt, "unit": "audio-s/s", "cores": _blas_threads(), "kind": "port",
               "sample": f"1 s (16 000 samples) of the same extraction (same weights), numpy oracle, 1 run after "
                         f"a warm-up, {cdt:.2f} s wall"}
    line = {
        "metric": "audio-sec pitch-extracted/sec (RMVPE, 10 s @16 kHz, 1 GPU)", "value": round(value, 2),
        "unit": "audio-s/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded glide + noise, random-init weights)",
        "config": {"workload": "rmvpe10s: RMVPE f0, 160000 samples @16 kHz -> f0 [1001], batch 1, fp32",
                   "samples": T, "frames": F, "batch": 1},
        "roofline": roofline, "cpu_baseline": cpu, "breakdown": breakdown,
    }
    print(json.dumps(line), flush=True)
    return 0


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="synth40k",
                    choices=("synth40k", "hubert", "dec48k-b8", "synth40k-bf16-b4", "synth40k-bf16rb-b4", "vc40k",
                             "rmvpe10s"),
                    help="synth40k: BASELINE config 2 (default); hubert: config 3; dec48k-b8: config 4; "
                         "synth40k-bf16-b4: config 5 (ups + enc_p matmuls on bf16); synth40k-bf16rb-b4: config 5 "
                         "with the ResBlocks on bf16 too (reported separately); vc40k: the conversion chain "
                         "HuBERT -> retrieval -> synthesis -> RMS mix -> int16 around config 2")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--quick", action="store_true",
                    help="only the timed steps (no per-family breakdown, host-I/O rate or CPU baseline); "
                         "for profiler runs")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="instead of the benchmark, run the library's plain copy kernel (rvc_copy) 5 times on "
                         "a MIB-sized buffer: the reference reading for the FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy)
    if args.gpus != 1:
        print(f"bench.py measures one MI355X only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    if args.workload == "hubert":
        return bench_hubert(args)
    if args.workload == "dec48k-b8":
        return bench_dec48(args)
    if args.workload == "rmvpe10s":
        return bench_rmvpe(args)
    if args.workload == "vc40k":
        return bench_vc(args)
    if args.workload.startswith("synth40k-bf16"):
        return bench_bf16(args, precision=1 if args.workload == "synth40k-bf16-b4" else 2)

    from rvc_hip import _hip, synthetic as syn
    from rvc_hip.hip_ops import get_context
    from rvc_hip.synth import HipSynthesizer

    if not _hip.has_so:
        raise RuntimeError(f"HIP backend missing: {_hip.so_load_error}")
    geom = syn.GEOM_40K
    w = syn.make_weights(geom, seed=0)
    ctx = get_context()
    s = HipSynthesizer(w, sr=geom.sr, ctx=ctx)
    _log(f"bench: device {_hip.device_name()}; weights resident")

    P, B = P_FRAMES, 1
    inp = syn.make_synth_inputs(geom, P, seed=3)
    ids = {
        "phone": ctx.upload(np.ascontiguousarray(inp["phone"], np.float32)),
        "pitch": ctx.upload(np.ascontiguousarray(inp["pitch"], np.int64)),
        "f0": ctx.upload(np.ascontiguousarray(inp["nsff0"], np.float32)),
        "sid": ctx.upload(np.ascontiguousarray(inp["sid"], np.int64)),
        "nz": ctx.upload(np.ascontiguousarray(inp["nz"], np.float32)),
        "ns": ctx.upload(np.ascontiguousarray(inp["ns"], np.float32).reshape(-1)),
    }
    n_out = P * geom.upp
    wave_id = ctx.alloc(B * n_out)

    def step():
        s.infer_dev(ids["phone"], ids["pitch"], ids["f0"], ids["sid"], ids["nz"], ids["ns"], B, P, wave_id)

    for _ in range(args.warmup):
        step()
    _log(f"bench: {args.warmup} warm-up steps done")

    # timed region; every step ends with a stream synchronize inside the call
    s.set_timing("dec.rb")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    dt = time.perf_counter() - t0
    rb = s.get_timing()
    s.set_timing("")
    ms_step = dt * 1e3 / args.steps
    audio_s = P / 100.0 * B
    value = audio_s * args.steps / dt
    _log(f"bench: {args.steps} steps, {ms_step:.3f} ms/step, {value:.1f} audio-s/s")

    # roofline of the dominant kernel family (the ResBlock MFMA convs, one launch per
    # dilation group and conv of each of the four stages: 24 launches per step)
    n_launch = max(rb["launches"], 1)
    avg_s = rb["ms"] / 1e3 / n_launch
    flops_launch = rb["flops"] / n_launch
    achieved = flops_launch / avg_s / 1e12 if avg_s > 0 else 0.0
    roofline = {"kernel": "conv1d_mfma (GeneratorNSF ResBlock convs, all stages)", "bound": "mfma",
                "achieved": round(achieved, 2), "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_FP32_TFLOPS, 4), "traffic": profiled_traffic(),
                "algorithmic_bytes": int(rb["bytes"] / n_launch),
                "traffic_source": os.path.relpath(TRAFFIC_PROFILE, ROOT),
                "avg_launch_us": round(avg_s * 1e6, 2), "launches_per_step": n_launch // args.steps,
                "share_of_step": round(rb["ms"] / (dt * 1e3), 3)}

    # per-family breakdown (one extra untimed step per family)
    breakdown = {}
    for tag in () if args.quick else ("dec.rb.s0", "dec.rb.s1", "dec.rb.s2", "dec.rb.s3", "dec.avg", "dec.ups", "dec.noise", "dec.post",
                "dec.sine", "dec.pre", "enc", "flow"):
        s.set_timing(tag)
        step()
        breakdown[tag] = family_entry(s.get_timing())
    s.set_timing("")

    # PCIe-inclusive rate (host numpy in -> host numpy out): the median of 20
    # calls after 3 warm-ups; reported beside the device-resident headline
    host_io = host_io_ms = None
    if not args.quick:
        call = lambda: s.infer_controlled(inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"], inp["nz"], inp["ns"])  # noqa: E731
        for _ in range(3):
            call()
        times = []
        for _ in range(20):
            t0 = time.perf_counter()
            call()
            times.append(time.perf_counter() - t0)
        host_io_ms = float(np.median(times)) * 1e3
        host_io = round(audio_s / (host_io_ms / 1e3), 2)

    cpu = None if (args.no_cpu_baseline or args.quick) else cpu_baseline(w, geom)
    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "audio-s/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded inputs, random-init weights)",
        "config": {"workload": "config 2: RVC v2 40k enc_p+flow+GeneratorNSF, 10 s (P=1000), batch 1, fp32",
                   "frames": P, "batch": B, "sample_rate": SR, "output_samples": n_out},
        "roofline": roofline, "cpu_baseline": cpu,
        "host_io_audio_s_per_s": host_io,
        "host_io_ms_median": None if host_io_ms is None else round(host_io_ms, 4),
        "breakdown": breakdown,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
