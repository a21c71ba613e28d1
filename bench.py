#!/usr/bin/env python
"""Benchmark of the HIP Conformer encoder on one MI355X.

Workload: the full 24-block encoder with every
linear in the 4-bit code + per-row level-table format, batch 1, on a synthetic
log-mel [17656, 128] (176.56 s of audio) -> T = 2207 encoder frames. One step =
conv front end + 24 blocks + projector over that utterance, with the mel
already resident in HBM. value = audio seconds per second (encoder RTFx),
over K steps that replay the encode's HIP graph (what a caller repeating one
packing gets), with no timing events in them.

Also reported:
  roofline     - the dominant kernel of the step (the largest time per step
                 in a separate pass that times every launch), from HIP events
                 attached to its dispatches on the library's stream in K more
                 steps run right after the timed region (launched one by one,
                 as events cannot ride on kernels inside a graph; every 8th
                 launch of it carries them);
  breakdown    - per-operator times from that separate all-launch pass;
  gemm_lowbit  - the isolated 4-bit linear of configs[1] (bf16 activations,
                 bf16 out) at T in {188, 2207}, rotating >256 MB of distinct
                 codes/activations so the MALL cannot serve them;
  mel_frontend - the GPU log-mel front end on the workload's 176.56 s of audio;
  tdt_decoder  - the greedy TDT decoder over a T = 2207 synthetic pooler in
                 HBM with synthetic decoder weights (ms per decode, tokens);
  pipeline_wave_to_tokens - the workload's wave from host memory through
                 log-mel, encoder and TDT decoder to tokens in one call;
  workloads    - configs[2] (T = 188, f16 weights; and the 4-bit encoder at
                 T = 188) with the weight-streaming HBM fraction, and
                 configs[4] (16 utterances of U(5, 60) s in one packed call;
                 the 20-minute T = 15000 stream with its attention roofline);
  roofline_runner_up - the second-largest operator's roofline from the
                 all-launch pass;
  cpu_baseline - the CPU oracle (C restatement of the reference CPU backend)
                 on this host's cores: by default the complete workload
                 (--cpu-blocks 24); fewer blocks time a sample and scale the
                 median block time to 24 blocks.
"""
from __future__ import annotations

import argparse
import importlib
import importlib.util
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
FRAMES = 17656
AUDIO_S = FRAMES * 0.01
PEAK_F16_TFLOPS = 2500.0  # MI355X dense f16/bf16 MFMA
PEAK_HBM_GBS = 8000.0
PROFILE_STEPS = 3  # steps of the all-operator breakdown pass


def load_pkg():
    name = "bark3_wgpu_amd"
    if name in sys.modules:
        return sys.modules[name]
    init = ROOT / "bark3-wgpu_amd" / "__init__.py"
    spec = importlib.util.spec_from_file_location(name, init, submodule_search_locations=[str(init.parent)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def bench_encoder(pkg, synth, torch, steps: int, warmup: int):
    src = synth.SynthCheckpoint(seed=0, n_layers=24, style="baseline", lowbit=True)
    t0 = time.time()
    # the decoder's weights ride along for the wave -> tokens pipeline measured
    # after the encoder (they do not touch the encoder step); the blank row's
    # bias is lowered so that the synthetic encoder's small outputs decode to a
    # mix of token and blank steps (with the default bias every step is blank)
    enc = pkg.HipEncoder.load_with(src, device=0, n_layers=24, decoder=synth.SynthTdt(seed=0, blank_bias=-1.0))
    log(f"[bench] weights loaded in {time.time() - t0:.1f}s")
    mel = torch.from_numpy(synth.mel(FRAMES, seed=0)).cuda()
    T = pkg.conv_len(pkg.conv_len(pkg.conv_len(FRAMES)))
    pooler = torch.empty((T, 640), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def step():
        enc.encode_mel_batch_device(mel.data_ptr(), [FRAMES], [FRAMES], pooler.data_ptr(), pooler.numel(), stream)

    for _ in range(max(warmup, 3)):  # the second call captures the HIP graph, later ones replay it
        step()
    torch.cuda.synchronize()
    assert bool(torch.isfinite(pooler).all()), "non-finite encoder output"
    # the timed region: K steps as a caller repeating this packing runs them
    # (HIP graph replays), no timing events
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    log(f"[bench] encoder step {dt * 1e3:.3f} ms over {steps} steps (T={T}, graph replays)")
    # per-operator breakdown: a separate pass with every launch bracketed
    # (launched one by one: events cannot ride on kernels inside a graph)
    enc.profile_only(None)
    enc.profile(True)
    for _ in range(PROFILE_STEPS):
        step()
    torch.cuda.synchronize()
    prof = enc.profile_report()
    # the dominant kernel (largest time per step): K more steps in which only
    # its launches carry events give its average launch time
    dom = max(prof, key=lambda k: prof[k]["ms"])
    enc.profile_only(dom)
    enc.profile(True)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    dt_ev = (time.perf_counter() - t1) / steps
    timed = enc.profile_report()[dom]
    timed["step_ms"] = dt_ev * 1e3
    enc.profile(False)
    log(f"[bench] {dom} launches timed over {steps} more steps ({dt_ev * 1e3:.3f} ms per step, launched one by one)")
    pipe = bench_pipeline(enc)
    return enc, dt, T, prof, dom, timed, pipe


def bench_pipeline(enc, reps: int = 3):
    """bark_hip_transcribe_wave_batch on the workload's 176.56 s wave from host
    memory: upload, log-mel, the 24-block encoder and the greedy TDT decode of
    the pooler in device memory, tokens back to the host. The synthetic
    encoder's outputs are small, so the decoder's biases decide its steps
    (the blank bias is set for a mix of token and blank steps)."""
    enc.set_mel_filters()
    wave = mel_wave()
    toks = enc.transcribe_wave_batch([wave])[0]
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        toks = enc.transcribe_wave_batch([wave])[0]
        times.append(time.perf_counter() - t0)
    ms = sorted(times)[len(times) // 2] * 1e3
    audio_s = wave.size / 16000.0
    log(f"[bench] wave -> tokens pipeline: {ms:.2f} ms for {audio_s:.2f} s of audio ({len(toks)} tokens)")
    return {"audio_s": audio_s, "ms": ms, "audio_s_per_s": audio_s / (ms / 1e3), "tokens": int(len(toks)),
            "includes": "host->device wave upload (11.3 MB), log-mel, 24-block encoder, TDT decode, tokens to host"}


# the isolated 4-bit linear's (T, K, N) shapes
GEMM_SHAPES = [(t, k, n) for t in (188, 2207) for k, n in ((1024, 4096), (4096, 1024), (1024, 3072))]


def bench_gemm(pkg, torch, T: int, K: int, N: int, reps: int = 192):
    """Average launch time of the isolated 4-bit linear over `reps` distinct
    buffer sets (codes + activations + outputs)."""
    g = torch.Generator(device="cuda").manual_seed(T * 7 + K + N)
    A = [torch.randn((T, K), device="cuda", generator=g).to(torch.bfloat16) for _ in range(reps)]
    codes = [torch.randint(0, 256, (N, K // 2), device="cuda", dtype=torch.uint8, generator=g) for _ in range(reps)]
    lut = [torch.sort(torch.randn((N, 16), device="cuda", generator=g) * 0.02, dim=1).values.half() for _ in range(reps)]
    C = [torch.empty((T, N), device="cuda", dtype=torch.bfloat16) for _ in range(reps)]
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream

    def launch(i):
        pkg.lowbit_linear(A[i].data_ptr(), 1, codes[i].data_ptr(), lut[i].data_ptr(), C[i].data_ptr(), 2, T, K, N, sp)

    for i in range(reps):
        launch(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        launch(i)
    e1.record(stream)
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) / 1e3 / reps
    F = 2.0 * T * K * N
    B = K * N / 2 + 32 * N + 2 * T * K + 2 * T * N
    del A, codes, lut, C
    torch.cuda.empty_cache()
    return {"T": T, "K": K, "N": N, "us": t * 1e6, "tflops": F / t / 1e12, "gbs": B / t / 1e9,
            "mfma_frac": F / t / 1e12 / PEAK_F16_TFLOPS, "hbm_frac": B / t / 1e9 / PEAK_HBM_GBS}


# Linear weights streamed by one encode: per block the FFN pair twice, qkv,
# out, pointwise 1 and 2 and the relative-position key projection
# (25,165,824 weights over 18,432 output rows); f16, or 4-bit codes plus a
# 16-entry f16 table per row.
BLOCK_WEIGHTS, BLOCK_ROWS = 25_165_824, 18_432


def weight_bytes(lowbit: bool) -> float:
    per = BLOCK_WEIGHTS / 2 + 32 * BLOCK_ROWS if lowbit else 2 * BLOCK_WEIGHTS
    return 24.0 * per


def timed_encodes(torch, step, reps: int) -> float:
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / reps


def bench_t188(enc, pkg, synth, torch, lowbit: bool, reps: int = 50):
    """configs[2] (f16 weights from a bf16 checkpoint) or its 4-bit variant:
    the 24-block encoder on a 15 s log-mel [1500, 128] -> T = 188, batch 1,
    mel in HBM. Repeats of one packing replay a captured HIP graph."""
    own = enc is None
    if own:
        src = synth.SynthCheckpoint(seed=0, n_layers=24, style="baseline", lowbit=lowbit)
        enc = pkg.HipEncoder.load_with(src, device=0, n_layers=24)
    frames = 1500
    mel = torch.from_numpy(synth.mel(frames, seed=2)).cuda()
    T = pkg.conv_len(pkg.conv_len(pkg.conv_len(frames)))
    out = torch.empty((T, 640), device="cuda")
    sp = torch.cuda.current_stream().cuda_stream

    def step():
        enc.encode_mel_batch_device(mel.data_ptr(), [frames], [frames], out.data_ptr(), out.numel(), sp)

    for _ in range(5):
        step()
    dt = timed_encodes(torch, step, reps)
    assert bool(torch.isfinite(out).all()), "non-finite encoder output"
    if own:
        enc.close()
    wb = weight_bytes(lowbit)
    return {"workload": ("BASELINE configs[2]: 24-block encoder, f16 weights (bf16 checkpoint), log-mel 1500x128 -> T=188"
                         if not lowbit else "configs[2] input through the 4-bit encoder of configs[3], T=188"),
            "T": T, "ms_per_encode": dt * 1e3, "audio_s_per_s": frames * 0.01 / dt, "reps": reps,
            "weight_bytes": wb, "weight_gbs": wb / dt / 1e9, "hbm_frac": wb / dt / 1e9 / PEAK_HBM_GBS}


def bench_batch16(enc, pkg, synth, torch, reps: int = 5):
    """16 utterances with lengths drawn uniformly from 5-60 s
    (seeded), packed into one batched encode (per-sequence masks in attention
    and the depthwise conv), mel in HBM."""
    rng = np.random.default_rng(4)
    secs = rng.uniform(5.0, 60.0, 16)
    frames = [int(round(x * 100)) for x in secs]
    mel = torch.from_numpy(np.concatenate([synth.mel(f, seed=100 + i) for i, f in enumerate(frames)])).cuda()
    ts = [pkg.conv_len(pkg.conv_len(pkg.conv_len(f))) for f in frames]
    out = torch.empty((sum(ts), 640), device="cuda")
    sp = torch.cuda.current_stream().cuda_stream

    def step():
        enc.encode_mel_batch_device(mel.data_ptr(), frames, frames, out.data_ptr(), out.numel(), sp)

    for _ in range(2):
        step()
    dt = timed_encodes(torch, step, reps)
    assert bool(torch.isfinite(out).all()), "non-finite encoder output"
    audio = sum(frames) * 0.01
    return {"workload": "BASELINE configs[4] batch: 16 utterances U(5,60) s (seed 4), 24-block 4-bit encoder, one packed call",
            "audio_s": audio, "frames": sum(frames), "T_total": sum(ts), "T_max": max(ts), "ms_per_batch": dt * 1e3,
            "audio_s_per_s": audio / dt, "reps": reps}


def bench_long_stream(enc, pkg, synth, torch, reps: int = 3):
    """configs[4] single stream: 20 minutes (log-mel [120000, 128]) -> T = 15000
    through the 24-block 4-bit encoder as one sequence; with the attention
    kernel's roofline from HIP events on its launches."""
    frames = 120000
    mel = torch.from_numpy(synth.mel(frames, seed=5)).cuda()
    T = pkg.conv_len(pkg.conv_len(pkg.conv_len(frames)))
    out = torch.empty((T, 640), device="cuda")
    sp = torch.cuda.current_stream().cuda_stream

    def step():
        enc.encode_mel_batch_device(mel.data_ptr(), [frames], [frames], out.data_ptr(), out.numel(), sp)

    step()
    dt = timed_encodes(torch, step, reps)
    assert bool(torch.isfinite(out).all()), "non-finite encoder output"
    enc.profile_only("rel_attention")
    enc.profile(True)
    step()
    torch.cuda.synchronize()
    a = enc.profile_report()["rel_attention"]
    enc.profile(False)
    enc.profile_only(None)
    avg = a["ms"] / a["count"] / 1e3
    tf = 6144.0 * T * T / avg / 1e12
    del mel, out
    torch.cuda.empty_cache()
    return {"workload": "BASELINE configs[4] stream: 20 min log-mel 120000x128 -> T=15000, 24-block 4-bit encoder",
            "T": T, "ms_per_encode": dt * 1e3, "audio_s_per_s": frames * 0.01 / dt, "reps": reps,
            "attention": {"avg_launch_us": avg * 1e6, "tflops": tf, "frac": tf / PEAK_F16_TFLOPS,
                          "flops_per_launch": 6144.0 * T * T}}


def mel_wave() -> "np.ndarray":
    """Synthetic 16 kHz wave whose log-mel has the encoder workload's 17656 frames."""
    n = 160 * (FRAMES - 1) + 100
    rng = np.random.default_rng(0)
    t = np.arange(n) / 16000.0
    return (0.2 * np.sin(2 * np.pi * (300 + 40 * t) * t) + 0.02 * rng.standard_normal(n)).astype(np.float32)


def bench_mel(pkg, torch, reps: int = 20):
    """GPU log-mel front end (bark_hip_mel_device) on the workload's audio, wave
    resident in HBM: per-call time from events attached to its kernels."""
    wave = mel_wave()
    enc = pkg.HipEncoder(0, 1)
    enc.set_mel_filters()
    d_w = torch.from_numpy(wave).cuda()
    nf = 1 + wave.size // 160
    d_out = torch.empty((nf, 128), dtype=torch.float32, device="cuda")
    sp = torch.cuda.current_stream().cuda_stream
    for _ in range(3):
        enc.mel_device(d_w.data_ptr(), wave.size, d_out.data_ptr(), d_out.numel(), sp)
    torch.cuda.synchronize()
    enc.profile(True)
    for _ in range(reps):
        enc.mel_device(d_w.data_ptr(), wave.size, d_out.data_ptr(), d_out.numel(), sp)
    torch.cuda.synchronize()
    rep = enc.profile_report()["mel"]
    enc.profile(False)
    enc.close()
    ms = rep["ms"] / rep["count"]
    byts = rep["bytes"] / rep["count"]
    return {"samples": int(wave.size), "frames": nf, "audio_s": wave.size / 16000.0, "gpu_ms": ms,
            "audio_s_per_s": wave.size / 16000.0 / (ms / 1e3), "gbs": byts / (ms / 1e3) / 1e9}


def cpu_mel(pkg) -> float:
    """The numpy oracle's log-mel of the same wave (ms)."""
    from oracle import mel as omel

    filters = importlib.import_module("bark3_wgpu_amd.mel").slaney_mel_filters()
    wave = mel_wave()
    t0 = time.perf_counter()
    omel.features(wave, filters)
    return (time.perf_counter() - t0) * 1e3


TDT_T = 2207  # encoder frames of the workload


def bench_tdt(pkg, synth, torch, reps: int = 5):
    """Greedy TDT decoder (bark_hip_tdt_decode_device) over a synthetic pooler
    of the workload's T frames resident in HBM, synthetic decoder weights
    (synth.SynthTdt): median wall time per decode (the call returns with the
    tokens in host memory)."""
    enc = pkg.HipEncoder.load_with(synth.SynthCheckpoint(seed=1, n_layers=1), 0, 1, front_end=False,
                                   decoder=synth.SynthTdt(seed=0))
    pooler = synth.pooler(TDT_T, 9)
    d_p = torch.from_numpy(pooler).cuda()
    sp = torch.cuda.current_stream().cuda_stream
    torch.cuda.synchronize()
    for _ in range(2):
        toks = enc.tdt_decode_device(d_p.data_ptr(), TDT_T, sp)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        toks = enc.tdt_decode_device(d_p.data_ptr(), TDT_T, sp)
        times.append(time.perf_counter() - t0)
    # eight utterances of the same length decoded together (every launch
    # advances all of them); pooler seeds 11, 17 and 18 are left out: with
    # these synthetic weights they fall into runs of duration-0 tokens that
    # only the step guard ends (~30k tokens), which no speech does
    batch = [synth.pooler(TDT_T, s) for s in (9, 10, 12, 13, 14, 15, 16, 19)]
    enc.tdt_decode_batch(batch)
    t0 = time.perf_counter()
    btoks = enc.tdt_decode_batch(batch)
    batch_ms = (time.perf_counter() - t0) * 1e3
    enc.close()
    ms = sorted(times)[len(times) // 2] * 1e3
    return {"T": TDT_T, "audio_s": AUDIO_S, "tokens": int(len(toks)), "ms": ms,
            "us_per_frame": ms * 1e3 / TDT_T, "audio_s_per_s": AUDIO_S / (ms / 1e3),
            "batch8": {"ms": batch_ms, "tokens": [int(len(x)) for x in btoks],
                       "audio_s_per_s": 8 * AUDIO_S / (batch_ms / 1e3)}}


def cpu_tdt(synth) -> dict:
    """The numpy oracle's decode of the same pooler (ms) and its step count."""
    from oracle import tdt as otdt

    d = otdt.Decoder(synth.SynthTdt(seed=0))
    t0 = time.perf_counter()
    toks, margins = d.decode(synth.pooler(TDT_T, 9), with_margins=True)
    return {"cpu_ms": (time.perf_counter() - t0) * 1e3, "steps": int(len(margins)), "cpu_tokens": int(len(toks))}


def cpu_baseline(synth, blocks: int):
    """Oracle timing on this host's cores. blocks == 24 runs the complete
    workload (front end over the 17656-frame mel, 24 blocks, projector);
    fewer blocks time a sample and extrapolate 24 x the median block time."""
    sys.path.insert(0, str(ROOT))
    import oracle

    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    src = synth.SynthCheckpoint(seed=0, n_layers=blocks, style="baseline", lowbit=True)
    enc = oracle.Encoder(src, n_layers=blocks)
    mel = synth.mel(FRAMES, seed=0)
    t0 = time.perf_counter()
    sub = oracle.subsample(src, mel, threads=threads)
    t_front = time.perf_counter() - t0
    T = sub.shape[0]
    if blocks == 24:
        t0 = time.perf_counter()
        enc.encode(sub, T, threads=threads)
        total = t_front + (time.perf_counter() - t0)
        sample = (f"complete workload: front end over {FRAMES} mel frames, 24 blocks at T={T}, projector; "
                  f"{total:.2f} s")
    else:
        sub_w = oracle.PackW(oracle.round_f16(src.read("encoder.subsampling.linear.weight")), half=True)
        t0 = time.perf_counter()
        x = oracle.gemm(sub, sub_w, threads=threads)
        t_lin = time.perf_counter() - t0
        per_block = []
        for l in range(blocks):
            t0 = time.perf_counter()
            x = enc.block(l, x, threads=threads)
            per_block.append(time.perf_counter() - t0)
        proj_w = oracle.PackW(oracle.round_f16(src.read("encoder_projector.weight")), half=True)
        t0 = time.perf_counter()
        oracle.gemm(x, proj_w, threads=threads)
        t_proj = time.perf_counter() - t0
        t_block = float(np.median(per_block))
        total = t_front + t_lin + 24 * t_block + t_proj
        sample = (f"front end over {FRAMES} mel frames + sub linear + {blocks} of 24 blocks at T={T} + projector; "
                  f"24-block time = 24 x median block {t_block:.3f} s; total {total:.2f} s")
    # calibration: the reference's CPU GEMM throughput shapes (src/cpu/gemm.rs
    # throughput test: f32 weights, m x n x k) through the oracle's GEMM
    gemm_rates = []
    for m, n, k in ((2208, 4096, 1024), (2240, 4096, 1024), (448, 4096, 1024), (191, 4096, 1024),
                    (191, 1024, 4096), (191, 3072, 1024)):
        a = np.full((m, k), 0.01, np.float32)
        w = oracle.PackW(np.full((n, k), 0.02, np.float32))
        oracle.gemm(a[:8], w, threads=threads)
        t0 = time.perf_counter()
        oracle.gemm(a, w, threads=threads)
        gemm_rates.append({"m": m, "n": n, "k": k, "gflops": 2.0 * m * n * k / (time.perf_counter() - t0) / 1e9})
    return {"value": AUDIO_S / total, "unit": "audio s/s", "cores": threads, "kind": "port", "sample": sample,
            "cpu_model": cpu_model(), "gemm_f32_throughput": gemm_rates}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def calibration_copy(torch) -> None:
    """A 512 MiB device-to-device copy: the counter passes scale FETCH_SIZE and
    WRITE_SIZE by what they read for its known bytes."""
    a = torch.empty(128 << 20, dtype=torch.float32, device="cuda")
    a.fill_(1.0)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    del a, b
    torch.cuda.empty_cache()


def gemm_workload(pkg, torch) -> None:
    """What the isolated-linear counter passes profile (rocprofv3 ... -- python3
    bench.py --gemm-workload): the calibration copy, then bench_gemm over the
    six configs[1] shapes in order, each launched 2 x 192 times over 192
    distinct buffer sets (warm-up pass, then the timed pass)."""
    calibration_copy(torch)
    for t, k, n in GEMM_SHAPES:
        r = bench_gemm(pkg, torch, t, k, n)
        log(f"[bench] lowbit linear T={t} K={k} N={n}: {r['us']:.2f} us")


def traffic_workload(pkg, synth, torch, t: int = 2207, f16: bool = False) -> None:
    """What the counter passes profile (rocprofv3 --pmc ... -- python3 bench.py
    --traffic-workload [--traffic-t T] [--traffic-f16]): a 512 MiB device copy
    whose bytes calibrate the traffic counters, then two encodes of a 1-block
    encoder (4-bit, or f16 weights) on a synthetic log-mel giving T encoder
    frames: front end, one block and projector, the per-layer launches of the
    24-block step."""
    calibration_copy(torch)
    frames = 8 * t
    while pkg.conv_len(pkg.conv_len(pkg.conv_len(frames))) > t:
        frames -= 1
    while pkg.conv_len(pkg.conv_len(pkg.conv_len(frames))) < t:
        frames += 1
    src = synth.SynthCheckpoint(seed=0, n_layers=1, style="baseline", lowbit=not f16)
    with pkg.HipEncoder.load_with(src, device=0, n_layers=1) as enc:
        mel = synth.mel(frames, seed=0)
        enc.encode_mel(mel)
        enc.encode_mel(mel)
    torch.cuda.synchronize()
    log(f"[bench] traffic workload done (T={t}, {'f16' if f16 else '4-bit'} weights, {frames} mel frames)")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-blocks", type=int, default=24)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--traffic-workload", action="store_true",
                    help="run only the workload of the counter passes")
    ap.add_argument("--traffic-t", type=int, default=2207, help="encoder frames of the counter workload")
    ap.add_argument("--traffic-f16", action="store_true", help="counter workload with f16 weights")
    ap.add_argument("--gemm-workload", action="store_true",
                    help="run only the isolated 4-bit linear's counter workload")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        return 2

    import torch

    pkg = load_pkg()
    synth = importlib.import_module("bark3_wgpu_amd.synth")
    if not torch.cuda.is_available() or pkg.lib().bark_hip_device_count() < 1:
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1

    if args.traffic_workload:
        traffic_workload(pkg, synth, torch, args.traffic_t, args.traffic_f16)
        return 0
    if args.gemm_workload:
        gemm_workload(pkg, torch)
        return 0

    enc, dt, T, prof, dom, d, pipe = bench_encoder(pkg, synth, torch, args.steps, args.warmup)
    workloads = {}
    workloads["configs4_batch16"] = bench_batch16(enc, pkg, synth, torch)
    workloads["configs4_t15000"] = bench_long_stream(enc, pkg, synth, torch)
    workloads["t188_lowbit"] = bench_t188(enc, pkg, synth, torch, lowbit=True)
    enc.close()
    workloads["configs2_t188_f16"] = bench_t188(None, pkg, synth, torch, lowbit=False)
    for k, v in workloads.items():
        log(f"[bench] {k}: " + ", ".join(f"{kk}={vv:.4g}" if isinstance(vv, float) else f"{kk}={vv}"
                                          for kk, vv in v.items() if not isinstance(vv, dict)))
    # roofline of the dominant kernel from its launches in the event pass that
    # follows the timed region (every profiled label is one kernel, so this is
    # rocprof's average duration)
    avg_s = d["ms"] / d["count"] / 1e3
    mfma_bound = d["flops"] > 0 and d["flops"] / d["bytes"] > PEAK_F16_TFLOPS / PEAK_HBM_GBS * 1e3
    if mfma_bound:
        per_launch, peak, unit = d["flops"] / d["count"], PEAK_F16_TFLOPS, "TFLOP/s"
        achieved = per_launch / avg_s / 1e12
    else:
        per_launch, peak, unit = d["bytes"] / d["count"], PEAK_HBM_GBS, "GB/s"
        achieved = per_launch / avg_s / 1e9
    # the runner-up's roofline from the all-launch pass
    second = sorted(prof, key=lambda k: -prof[k]["ms"])[1] if len(prof) > 1 else None
    runner_up = None
    if second is not None:
        r = prof[second]
        r_avg = r["ms"] / r["count"] / 1e3
        r_mfma = r["flops"] > 0 and r["flops"] / r["bytes"] > PEAK_F16_TFLOPS / PEAK_HBM_GBS * 1e3
        r_ach = (r["flops"] / r["count"] / r_avg / 1e12) if r_mfma else (r["bytes"] / r["count"] / r_avg / 1e9)
        r_peak = PEAK_F16_TFLOPS if r_mfma else PEAK_HBM_GBS
        runner_up = {"kernel": second, "bound": "mfma" if r_mfma else "hbm", "achieved": r_ach, "peak": r_peak,
                     "unit": "TFLOP/s" if r_mfma else "GB/s", "frac": r_ach / r_peak, "avg_launch_us": r_avg * 1e6,
                     "timing": "all-launch breakdown pass"}
    breakdown = {k: {"ms_per_step": v["ms"] / PROFILE_STEPS, "launches_per_step": v["count"] // PROFILE_STEPS,
                     "tflops": (v["flops"] / (v["ms"] / 1e3) / 1e12) if v["flops"] else None,
                     "gbs": v["bytes"] / (v["ms"] / 1e3) / 1e9}
                 for k, v in sorted(prof.items(), key=lambda kv: -kv[1]["ms"])}
    log(f"[bench] breakdown (separate pass, every launch timed; sum {sum(v['ms_per_step'] for v in breakdown.values()):.3f} ms/step):")
    for k, v in breakdown.items():
        log(f"[bench]   {k:16s} {v['ms_per_step']:8.3f} ms/step  x{v['launches_per_step']:<4d} "
            f"{(v['tflops'] or 0):8.1f} TFLOP/s {v['gbs']:8.1f} GB/s")

    traffic = None
    tfile = ROOT / "profiles" / "traffic.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get(dom)

    gemm = []
    if not args.no_gemm:
        for t, k, n in GEMM_SHAPES:
            r = bench_gemm(pkg, torch, t, k, n)
            gemm.append(r)
            log(f"[bench] lowbit linear T={t} K={k} N={n}: {r['us']:.2f} us, {r['tflops']:.1f} TFLOP/s, "
                f"{r['gbs']:.0f} GB/s")

    mel = bench_mel(pkg, torch)
    log(f"[bench] log-mel front end: {mel['gpu_ms']:.3f} ms for {mel['audio_s']:.2f} s of audio "
        f"({mel['audio_s_per_s']:.0f} audio s/s)")

    tdt = bench_tdt(pkg, synth, torch)
    log(f"[bench] TDT decode: {tdt['ms']:.2f} ms for T={tdt['T']} ({tdt['tokens']} tokens, "
        f"{tdt['us_per_frame']:.1f} us/frame, {tdt['audio_s_per_s']:.0f} audio s/s)")

    cpu = None
    if not args.no_cpu:
        tdt.update(cpu_tdt(synth))
        tdt["cpu_kind"] = "port (numpy oracle, oracle/tdt.py, float64)"
        log(f"[bench] TDT decode on the CPU oracle: {tdt['cpu_ms']:.1f} ms ({tdt['steps']} steps)")
        mel["cpu_ms"] = cpu_mel(pkg)
        mel["cpu_kind"] = "port (numpy oracle, oracle/mel.py)"
        log(f"[bench] log-mel on the CPU oracle: {mel['cpu_ms']:.1f} ms")
        t0 = time.time()
        cpu = cpu_baseline(synth, args.cpu_blocks)
        log(f"[bench] cpu baseline {cpu['value']:.2f} audio s/s ({time.time() - t0:.1f}s)")

    line = {
        "metric": "encoder RTFx (audio s/s), 24-block 4-bit Conformer encoder, 1 GPU",
        "value": AUDIO_S / dt,
        "unit": "audio s/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": dt * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded log-mel N(0,1); random-init weights, 4-bit codes U{0..15} + sorted N(0,0.02) f16 tables)",
        "config": {"workload": "BASELINE configs[3]: 24-block 4-bit encoder, log-mel 17656x128 -> T=2207, batch 1",
                   "frames": FRAMES, "T": T, "audio_s": AUDIO_S, "encoder_frames_per_s": T / dt,
                   "relative_keys": "every layer's relK (position table x relative_k_proj) is computed when "
                                    "the position table grows (the first encode of a new maximum length, "
                                    "in warmup here) and read by later encodes"},
        "roofline": {"kernel": dom, "bound": "mfma" if mfma_bound else "hbm", "achieved": achieved, "peak": peak,
                     "unit": unit, "frac": achieved / peak, "traffic": traffic,
                     ("flops_per_launch" if mfma_bound else "bytes_per_launch"): per_launch,
                     "avg_launch_us": avg_s * 1e6, "rule": "largest ms per step",
                     "timing": f"events on its {d['count']} launches in {args.steps} steps run right after the "
                               f"timed region ({d['step_ms']:.3f} ms per step, launched one by one)"},
        "roofline_runner_up": runner_up,
        "workloads": workloads,
        "breakdown": breakdown,
        "gemm_lowbit": gemm,
        "mel_frontend": mel,
        "tdt_decoder": tdt,
        "pipeline_wave_to_tokens": pipe,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
