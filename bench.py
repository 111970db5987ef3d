"""Benchmark of the MetalNN hot path on one MI355X: ms per 7.8 s stereo chunk.

One step = the HTDemucs-shaped time encoder (config 4) on 4 chunks, one chunk per forward
(batch 1, as the configuration is quoted), plus the cross-domain transformer bottleneck
(config 5) on those 4 chunks as one batch-4 forward. value = ms_per_step / 4
= t(config 4, batch 1) + t(config 5, batch 4) / 4, the headline metric. Inputs and weights are
seeded synthetic data of the configurations' shapes, resident in HBM before timing starts.

The headline is the wall clock around the K timed steps. Per-kernel-family GPU time comes from a
second pass of K steps with HIP events bracketing every library launch on its stream
(mnn_device_kernel_timing); the dominant family is reported against MI355X peak as `roofline`,
every family (the encoder's per level) in `kernels`. The CPU baseline times the torch-CPU
restatement of the same layers (oracle/torch_cpu.py) on one chunk on the host cores.

Usage: python bench.py [--gpus 1] [--steps 10] [--warmup 3] [--precision f32|bf16]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "ms per 7.8s stereo chunk (HTDemucs-shaped); per-kernel % of HBM/MFMA roofline"
PEAK = {"hbm": 8.0e12, "f32": 157.3e12, "bf16": 2.5e15}  # B/s, FLOP/s (MI355X datasheet, dense)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Markers:
    """roctx ranges around the bench's passes, so that a `rocprofv3 --marker-trace` run can
    attribute kernel dispatches to them (metalaudio_amd.profsummary trace --range ...). No-ops when
    the marker library is absent."""

    def __init__(self):
        import ctypes
        self.lib = None
        for name in ("librocprofiler-sdk-roctx.so.1", "/opt/rocm/lib/librocprofiler-sdk-roctx.so.1",
                     "libroctx64.so", "/opt/rocm/lib/libroctx64.so"):
            try:
                self.lib = ctypes.CDLL(name)
                break
            except OSError:
                continue

    def push(self, msg):
        if self.lib:
            self.lib.roctxRangePushA(msg.encode())

    def pop(self):
        if self.lib:
            self.lib.roctxRangePop()


# ------------------------------------------------------------------ algorithmic work per step
def encoder_work(gn=True, gn_l1=None):
    """Algorithmic flops and bytes per chunk of config 4, per encoder kernel and level (the
    kernel-timing names carry the level's channel count, e.g. "enc_conv_f32[c96]").
    bytes = inputs read once + outputs written once + weights once; flops = 2 M N K.
    gn: the one-launch GroupNorm form of levels 2-4 (the split-K finish applies GroupNorm + GELU);
    gn_l1 (default gn): the first level in one pass; else the two-pass forms."""
    if gn_l1 is None:
        gn_l1 = gn
    import ctypes
    from metalaudio_amd import workloads as W
    from metalaudio_amd._lib import lib
    L = W.CHUNK_SAMPLES
    fam = {}
    ch = W.ENC_CHANNELS

    def add(name, flops, byts):
        f = fam.setdefault(name, [0.0, 0.0])
        f[0] += flops
        f[1] += byts
    for i in range(4):
        cin, cout = ch[i], ch[i + 1]
        lo = (L + 6 - 8) // 4 + 1
        conv_flops = 2.0 * cout * lo * cin * 8
        rw_flops = 2.0 * 2 * cout * lo * cout
        x_b, y_b = 4.0 * cin * L, 4.0 * cout * lo
        conv_w = 4.0 * (cout * cin * 8 + cout)
        rw_w = 4.0 * (2 * cout * cout + 2 * cout)
        tag = f"[c{cout}]"
        if cin <= 4 and cout == 48 and gn_l1:
            # first level in one pass: conv, GroupNorm exchange, GELU, rewrite, GLU (x read once,
            # block output written)
            add("enc_l1_oneshot_f32" + tag, conv_flops + rw_flops, x_b + y_b + conv_w + rw_w)
        elif cin <= 4 and cout == 48:
            # fused first level: statistics pass (conv recomputed, x read) and the fused pass
            # (conv again + rewrite; x read, block output written)
            add("enc_l1_stats_f32" + tag, conv_flops, x_b + conv_w)
            add("enc_l1_fused_f32" + tag, conv_flops + rw_flops, x_b + y_b + conv_w + rw_w)
        else:
            sp, tm, tn = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
            lib().mnn_debug_enc_conv_plan(cin, cout, lo, 1, int(gn), ctypes.byref(sp),
                                          ctypes.byref(tm), ctypes.byref(tn))
            if gn:
                # the conv writes one partial product per K part; the finish sums them and writes
                # GELU(GroupNorm(y))^T, the rewrite reads it
                add("enc_conv_f32" + tag, conv_flops, x_b + conv_w + sp.value * y_b)
                add("enc_conv_reduce_gn_f32" + tag, 0.0, sp.value * y_b + y_b)
                add("enc_rewrite_f32" + tag, rw_flops, 2 * y_b + rw_w)
                L = lo
                continue
            if sp.value > 1:
                # the conv writes one partial product per K part, the reduce pass sums them
                add("enc_conv_f32" + tag, conv_flops, x_b + conv_w + sp.value * y_b)
                add("enc_conv_reduce_f32" + tag, 0.0, sp.value * y_b + y_b)
            else:
                add("enc_conv_f32" + tag, conv_flops, x_b + y_b + conv_w)
            add("enc_gn_gelu_t_f32" + tag, 0.0, 2 * y_b)  # y read, GELU(GN(y)) written
            add("enc_rewrite_f32" + tag, rw_flops, 2 * y_b + rw_w)
        L = lo
    return fam


def transformer_work(batch):
    from metalaudio_amd import workloads as W
    E, H, Hd, St, Sf = W.T5_EMBED, W.T5_HEADS, W.T5_FFN, W.T5_TIME_LEN, W.T5_FREQ_LEN
    hd = E // H
    attn_f = attn_b = gemm_f = gemm_b = ln_b = 0.0
    for i in range(W.T5_LAYERS):
        cross = i % 2 == 1
        for own, other in ((St, Sf), (Sf, St)):
            sk = other if cross else own
            attn_f += 4.0 * own * sk * hd * H * batch
            attn_b += 4.0 * batch * (own * E + 2 * sk * E + own * E)
            if cross:
                gemm_f += 2.0 * batch * (own * E * E + other * E * 2 * E)
            else:
                gemm_f += 2.0 * batch * own * E * 3 * E
            gemm_f += 2.0 * batch * own * (E * E + 2 * E * Hd)
            gemm_b += 4.0 * batch * own * (E + 3 * E + E + E + E + Hd + Hd + E)
            # LayerNorms folded into the GEMMs (fp32, E % 64 == 0): the residual GEMMs write
            # (mean, M2) per 64 columns of each row, the consumer GEMMs read them
            gemm_b += 8.0 * batch * (E // 64) * (own * 2 + (own + other if cross else own) + own)
            # standalone LayerNorms (the unfolded form): self layer two (read + write each);
            # cross layer the two normalisations of this state in one pass (one read, two
            # writes), then the feed-forward norm
            ln_b += 4.0 * batch * own * E * (5 if cross else 4)
    # the inputs' row statistics, with the copy of each input to its output
    parts_b = sum(batch * s * (8.0 * E + 8.0 * (E // 64)) for s in (St, Sf))
    return {"attn_fwd_f32": [attn_f, attn_b], "gemm_f32_mfma_nk": [gemm_f, gemm_b],
            "layernorm": [0.0, ln_b], "ln_row_parts_f32": [0.0, parts_b]}


# ------------------------------------------------------------------ model setup
def build_models(nn, W, dev, precision):
    c4 = W.config4()
    blocks = []
    seq = nn.Sequential(dev)
    for cin, cout, lv in zip(W.ENC_CHANNELS[:-1], W.ENC_CHANNELS[1:], c4["levels"]):
        b = nn.UNetEncoderBlock(dev, cin, cout, 8, 4, 1, rewrite=True, precision=precision)
        b.load_weights(lv["conv.weight"], lv["conv.bias"], lv["norm.weight"], lv["norm.bias"],
                       lv["rewrite.weight"], lv["rewrite.bias"])
        blocks.append(b)
        seq.add(b)
    seq.build()
    c5 = W.config5(batch=W.T5_BATCH)
    ct = nn.CrossTransformerEncoder(dev, c5["embed"], c5["heads"], c5["ffn"], c5["layers"],
                                    c5["layer_scale"], precision=precision)
    ct.load_state(c5["params"])
    # 4 distinct chunks for the encoder, resident in HBM
    rng = np.random.Generator(np.random.PCG64(2024))
    chunks = [nn.Tensor.from_numpy(dev, c4["x"])]
    for _ in range(3):
        chunks.append(nn.Tensor.from_numpy(
            dev, rng.uniform(-1, 1, c4["x"].shape).astype(np.float32)))
    t_in = nn.Tensor.from_numpy(dev, c5["time"])
    f_in = nn.Tensor.from_numpy(dev, c5["freq"])
    t_out = nn.Tensor(dev, t_in.shape)
    f_out = nn.Tensor(dev, f_in.shape)
    return dict(seq=seq, blocks=blocks, ct=ct, chunks=chunks, t_in=t_in, f_in=f_in,
                t_out=t_out, f_out=f_out, c4=c4, c5=c5)


def run_encoder(m, stream):
    for x in m["chunks"]:
        m["seq"].forward(x, stream)


def run_transformer(m, stream):
    m["ct"].forward_cross(m["t_in"], m["f_in"], m["t_out"], m["f_out"], stream)


def timed(fn, stream, steps):
    stream.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    stream.sync()
    return (time.perf_counter() - t0) * 1e3 / steps


# ------------------------------------------------------------------ CPU baseline
def cpu_baseline(m, warmup=3, runs=10, budget_s=40.0):
    """The reference CPU path's stand-in: the torch-CPU restatement of the same layers
    (oracle/torch_cpu.py; the reference's Accelerate layers need Swift and Apple frameworks) on
    one chunk: config 4 at batch 1 and config 5 at batch 1 (the per-chunk share of the batch-4
    transformer), fp32, torch.inference_mode, all host threads; 3 warm-ups, then the median of
    10 runs (fewer if a run is so slow that 10 would exceed the budget)."""
    import platform

    import torch
    from metalaudio_amd import workloads as W
    from oracle import torch_cpu as tc
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    c4 = m["c4"]
    c5 = W.config5(batch=1)
    x = tc.to_torch(c4["x"])
    lv = [{k: tc.to_torch(v) for k, v in l.items()} for l in c4["levels"]]
    t = tc.to_torch(c5["time"])
    f = tc.to_torch(c5["freq"])
    p = {k: tc.to_torch(v) for k, v in c5["params"].items()}

    def one():
        with torch.inference_mode():
            tc.time_encoder(x, lv)
            tc.cross_transformer(t, f, p, c5["layers"], c5["heads"])
    for _ in range(warmup):
        one()
    times = []
    t_start = time.perf_counter()
    for _ in range(runs):
        t0 = time.perf_counter()
        one()
        times.append((time.perf_counter() - t0) * 1e3)
        if time.perf_counter() - t_start > budget_s:
            break
    cpu_model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(statistics.median(times), 2),
        "unit": "ms per chunk",
        "cores": int(threads),
        "kind": "port",
        "sample": f"median of {len(times)} runs after {warmup} warm-ups of one 7.8 s chunk: "
                  f"config 4 (batch 1) + config 5 at batch 1, torch-CPU restatement "
                  f"(oracle/torch_cpu.py), fp32, torch {torch.__version__}, "
                  f"{threads} threads, CPU: {cpu_model}",
    }


# ------------------------------------------------------------------ per-configuration table
def time_gpu(fn, stream, reps=50, warmup=5, sample_ms=0.1):
    """GPU ms of one call: `warmup` calls, then `reps` samples, each a few calls back to back
    bracketed by two timing marks (HIP events) on the stream, as many calls as make a sample of
    about sample_ms (a mark pair costs a few microseconds, which would dominate a short call
    timed alone); the median over the samples of their time per call."""
    import ctypes
    from metalaudio_amd._lib import check, lib
    ms = ctypes.c_float()

    def samples(n, calls):
        for i in range(n):
            check(lib().mnn_debug_stream_mark(stream.handle, 2 * i))
            for _ in range(calls):
                fn()
            check(lib().mnn_debug_stream_mark(stream.handle, 2 * i + 1))
        stream.sync()
        ts = []
        for i in range(n):
            check(lib().mnn_debug_stream_mark_elapsed(stream.handle, 2 * i, 2 * i + 1,
                                                      ctypes.byref(ms)))
            ts.append(ms.value / calls)
        return ts
    for _ in range(warmup):
        fn()
    stream.sync()
    est = statistics.median(samples(3, 1))
    calls = int(min(20, max(1, -(-sample_ms // max(est, 1e-4)))))
    time_gpu.calls = calls
    return statistics.median(samples(reps, calls))


class Floors:
    """Measured floors for bandwidth-bound rows: one launch of the library's streaming kernel
    (mnn_debug_stream_rw) reading and writing the row's algorithmic bytes, timed like the row
    (event-timed median of 50), and an empty launch. A row's kernel time over its floor says how
    far it is from what that traffic costs in one launch on this device."""

    def __init__(self, nn, dev, stream, max_bytes=40 << 20):
        from metalaudio_amd._lib import check, lib
        self.check, self.lib, self.stream = check, lib, stream
        n = max_bytes // 4
        self.src = nn.Tensor.from_numpy(dev, np.ones(n, np.float32))
        self.dst = nn.Tensor(dev, (n,))
        self.empty_us = round(time_gpu(lambda: check(lib().mnn_debug_empty_launch(stream.handle)),
                                       stream) * 1e3, 2)

    def of(self, read_bytes, write_bytes, gpu_ms):
        rd, wr = int(read_bytes) // 16 * 16, int(write_bytes) // 16 * 16

        def fn():
            self.check(self.lib().mnn_debug_stream_rw(self.src.handle, rd, self.dst.handle, wr,
                                                      self.stream.handle))
        us = time_gpu(fn, self.stream) * 1e3
        return {"us": round(us, 2), "read_bytes": rd, "write_bytes": wr,
                "empty_launch_us": self.empty_us, "frac_of_floor": round(us / (gpu_ms * 1e3), 4)}


def kernel_table(dev):
    """{kernel name: (launches, total ms)} of the device's kernel timing (exact names)."""
    import ctypes
    from metalaudio_amd._lib import check, lib
    need = ctypes.c_size_t()
    check(lib().mnn_debug_kernel_timing_table(dev.handle, None, 0, ctypes.byref(need)))
    buf = ctypes.create_string_buffer(need.value)
    check(lib().mnn_debug_kernel_timing_table(dev.handle, buf, need.value, ctypes.byref(need)))
    out = {}
    for line in buf.value.decode().splitlines():
        name, n, ms = line.rsplit(" ", 2)
        out[name] = (int(n), float(ms))
    return out


def kernel_breakdown(dev, stream, fn, reps=10, work=None, prec="f32"):
    """Per-kernel GPU time of one call (kernel-timing pass: every launch bracketed by events on
    its stream, `reps` calls): microseconds and launches per call, share of the call's kernel
    time and, where `work` gives the kernel's algorithmic flops or bytes per call, its fraction
    of the MFMA or HBM peak."""
    fn()
    stream.sync()
    dev.reset_kernel_timing()
    dev.set_kernel_timing(True)
    for _ in range(reps):
        fn()
    stream.sync()
    dev.set_kernel_timing(False)
    tab = kernel_table(dev)
    dev.reset_kernel_timing()
    total = sum(ms for _, ms in tab.values()) or 1.0
    out = {}
    for name, (n, ms) in sorted(tab.items(), key=lambda kv: -kv[1][1]):
        t = ms / reps * 1e-3  # seconds per call
        r = {"us": round(t * 1e6, 2), "launches": round(n / reps, 2),
             "share": round(ms / total, 4)}
        w = (work or {}).get(name)
        if w:
            flops, byts = w
            if flops:
                r["mfma_frac"] = round(flops / t / PEAK[prec], 4)
            if byts:
                r["hbm_frac"] = round(byts / t / PEAK["hbm"], 4)
        out[name] = r
    return out


def time_cpu(fn, budget_s=3.0, max_reps=5):
    ts = []
    t_start = time.perf_counter()
    while len(ts) < max_reps and (not ts or time.perf_counter() - t_start < budget_s):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(ts)


DEC_LEVELS = [(384, 192, 1344, 8), (192, 96, 5376, 8), (96, 48, 21504, 8), (48, 2, 86016, 2)]


def decoder_setup(nn, dev):
    """UNetDecoderBlock levels of the time branch (in = skip channels, out channels, input
    length, groups), seeded synthetic weights, inputs and skips."""
    r = np.random.default_rng(1006)
    blocks, skips, outs, params, flops = [], [], [], [], 0.0
    work = {}
    x = r.standard_normal((1, DEC_LEVELS[0][0], DEC_LEVELS[0][2])).astype(np.float32)
    for cin, cout, L, g in DEC_LEVELS:
        w = (r.standard_normal((2 * cin, cout, 8)) * np.sqrt(2.0 / (2 * cin * 2))).astype(np.float32)
        b = np.zeros(cout, np.float32)
        gm, bt = np.ones(cout, np.float32), np.zeros(cout, np.float32)
        sk = r.standard_normal((1, cin, L)).astype(np.float32)
        blk = nn.UNetDecoderBlock(dev, cin, cin, cout, 8, 4, g)
        blk.load_weights(w, b, gm, bt)
        blocks.append(blk)
        skips.append(nn.Tensor.from_numpy(dev, sk))
        outs.append(nn.Tensor(dev, (1, cout, 4 * L)))
        params.append((w, b, gm, bt, g, sk))
        lf = 2.0 * 2 * cin * cout * 8 * L
        flops += lf
        # per kernel family: the matrix-core levels (transposed conv as a GEMM over the unfolded
        # [input; skip], 2 taps per phase) and the few-channel last level; GroupNorm apply reads
        # and writes the output once
        if cout >= 8:
            _acc(work, "convt_f32_mfma", lf, 0)
            _acc(work, "convt_pack_f32", 0, 4.0 * 2 * cin * L * (1 + 2))
        else:
            _acc(work, "convt_small_f32", lf, 4.0 * (2 * cin * L + cout * 4 * L))
        _acc(work, "gn_apply_parts", 0, 8.0 * cout * 4 * L)
    return {"blocks": blocks, "skips": skips, "outs": outs, "params": params, "flops": flops,
            "work": work, "x": nn.Tensor.from_numpy(dev, x), "x_host": x}


def _acc(work, name, flops, byts):
    w = work.setdefault(name, [0.0, 0.0])
    w[0] += flops
    w[1] += byts


def decoder_oracle(oracle, dec):
    y = dec["x_host"]
    for w, b, gm, bt, g, sk in dec["params"]:
        y = oracle.decoder_block(y, sk, w, b, gm, bt, g, dtype=np.float32)
    return y


# Frequency branch as the reference's HTDemucs builds it (HTDemucs.swift:295-331): stereo
# magnitude spectrogram of a 7.8 s chunk, nfft 4096 -> 2049 bins padded to 2064 (a multiple of
# 2^4, UNetPaddingCalculator2D) x 336 frames; 3x3 kernels, stride (2, 2), channels
# 2 -> 48 -> 96 -> 192 -> 384, GroupNorm min(8, C) groups; decoders mirror with skips.
FREQ_CH = [2, 48, 96, 192, 384]
FREQ_BINS, FREQ_FRAMES = 2064, 336


def freq_setup(nn, dev):
    """FreqUNetEncoderBlock2D levels down and FreqUNetDecoderBlock2D levels back up (skips of
    the encoder's shapes), seeded synthetic weights and inputs."""
    r = np.random.default_rng(1007)
    enc = {"blocks": [], "outs": [], "params": [], "flops": 0.0, "work": {}}
    dec = {"blocks": [], "skips": [], "outs": [], "params": [], "flops": 0.0, "work": {}}
    H, W = FREQ_BINS, FREQ_FRAMES
    x = r.standard_normal((1, FREQ_CH[0], H, W)).astype(np.float32)
    dims = []
    for i in range(4):
        cin, cout = FREQ_CH[i], FREQ_CH[i + 1]
        g = min(8, cin) if i == 0 else 8
        g = min(8, cout) if cout < 8 else g
        w = (r.standard_normal((cout, cin, 3, 3)) * np.sqrt(2.0 / (9 * cin))).astype(np.float32)
        b = np.zeros(cout, np.float32)
        gm, bt = np.ones(cout, np.float32), np.zeros(cout, np.float32)
        blk = nn.FreqUNetEncoderBlock2D(dev, cin, cout, 3, 2, g)
        blk.load_weights(w, b, gm, bt)
        dims.append((H // 2, W // 2))
        enc["blocks"].append(blk)
        enc["outs"].append(nn.Tensor(dev, (1, cout, H // 2, W // 2)))
        enc["params"].append((w, b, gm, bt, g))
        lf = 2.0 * cout * cin * 9 * (H // 2) * (W // 2)
        enc["flops"] += lf
        ho_wo = (H // 2) * (W // 2)
        if cin <= 2:  # direct register-window level (also writes the GroupNorm partials)
            _acc(enc["work"], "conv2d_small_f32", lf, 4.0 * (cin * H * W + cout * ho_wo))
        elif cin % 4 == 0 and cout % 96 == 0:  # implicit GEMM over LDS-staged input windows
            _acc(enc["work"], "conv2d_igemm_f32", lf, 0)
        else:  # unfolded operand (written once) + matrix-core GEMM
            _acc(enc["work"], "conv2d_f32_mfma", lf, 0)
            _acc(enc["work"], "conv2d_unfold_f32", 0, 4.0 * (cin * H * W + 9 * cin * ho_wo))
        _acc(enc["work"], "gn_apply_parts", 0, 8.0 * cout * ho_wo)
        H, W = H // 2, W // 2
    for i in reversed(range(4)):
        cin, cout = FREQ_CH[i + 1], FREQ_CH[i]
        g = min(8, cout)
        h, w_ = dims[i]
        w = (r.standard_normal((2 * cin, cout, 3, 3)) * np.sqrt(2.0 / (2 * cin * 9 / 4))).astype(
            np.float32)
        b = np.zeros(cout, np.float32)
        gm, bt = np.ones(cout, np.float32), np.zeros(cout, np.float32)
        sk = r.standard_normal((1, cin, h, w_)).astype(np.float32)
        blk = nn.FreqUNetDecoderBlock2D(dev, cin, cin, cout, 3, 2, g)
        blk.load_weights(w, b, gm, bt)
        dec["blocks"].append(blk)
        dec["skips"].append(nn.Tensor.from_numpy(dev, sk))
        dec["outs"].append(nn.Tensor(dev, (1, cout, 2 * h, 2 * w_)))
        dec["params"].append((w, b, gm, bt, g, sk))
        lf = 2.0 * 2 * cin * cout * 9 * h * w_
        dec["flops"] += lf
        if cout >= 8:  # tap GEMM over [input; skip], then the gather of the taps
            _acc(dec["work"], "convt2d_f32_mfma", lf, 0)
            if (h * w_) % 4:  # the GEMM reads them in place unless rows are not 16-byte multiples
                _acc(dec["work"], "convt_pack_f32", 0, 4.0 * 2 * cin * h * w_ * 2)
            _acc(dec["work"], "convt2d_gather_f32", 0, 4.0 * (9 * cout * h * w_ + cout * 4 * h * w_))
        else:
            _acc(dec["work"], "convt2d_small_f32", lf, 4.0 * (2 * cin * h * w_ + cout * 4 * h * w_))
        _acc(dec["work"], "gn_apply_parts", 0, 8.0 * cout * 4 * h * w_)
    enc["x"], enc["x_host"] = nn.Tensor.from_numpy(dev, x), x
    xd = r.standard_normal((1, FREQ_CH[-1], H, W)).astype(np.float32)
    dec["x"], dec["x_host"] = nn.Tensor.from_numpy(dev, xd), xd
    return enc, dec


def freq_encoder_oracle(oracle, enc):
    y = enc["x_host"]
    for w, b, gm, bt, g in enc["params"]:
        y = oracle.freq_encoder_block(y, w, b, gm, bt, g, dtype=np.float32)
    return y


def freq_decoder_oracle(oracle, dec):
    y = dec["x_host"]
    for w, b, gm, bt, g, sk in dec["params"]:
        y = oracle.freq_decoder_block(y, sk, w, b, gm, bt, g, dtype=np.float32)
    return y


def long_audio_setup():
    """The long-audio row's model: the reference's default time-domain HTDemucs (5 levels,
    48..768 channels, k 8, s 4, 4 stems, 8 groups) with seeded synthetic weights in the
    Separator's state-dict naming; returns (generator for the audio, config, state)."""
    r11 = np.random.default_rng(1009)
    ch11 = [48, 96, 192, 384, 768]
    cfg11 = {"input_channels": 2, "num_stems": 4, "channels": ch11, "kernel_size": 8,
             "stride": 4, "num_groups": 8}
    P11, chans = {}, [2] + ch11
    for i in range(5):
        ci, co = chans[i], chans[i + 1]
        P11[f"time_encoder.{i}"] = {
            "conv.weight": (r11.standard_normal((co, ci, 8)) * np.sqrt(2 / (8 * ci))).astype(
                np.float32), "conv.bias": np.zeros(co, np.float32),
            "norm.weight": np.ones(co, np.float32), "norm.bias": np.zeros(co, np.float32)}
    for j in range(5):
        i = 4 - j
        ci, co = chans[i + 1], (2 if i == 0 else chans[i])
        P11[f"time_decoder.{j}"] = {
            "conv_transpose.weight": (r11.standard_normal((2 * ci, co, 8)) * np.sqrt(
                1 / (4 * ci))).astype(np.float32), "conv_transpose.bias": np.zeros(co, np.float32),
            "norm.weight": np.ones(co, np.float32), "norm.bias": np.zeros(co, np.float32)}
    for h in range(4):
        P11[f"output_heads.{h}"] = {"weight": r11.standard_normal((2, 2, 1)).astype(np.float32),
                                    "bias": np.zeros(2, np.float32)}
    return r11, cfg11, P11


def next_rows(nn, dev, stream):
    """Rows 6-10 of the configuration table, the hot path's next rows, on synthetic inputs:
    name -> {fn (one call), flops or byts (algorithmic), floor (read, write bytes) for the
    bandwidth-bound rows, work (per-kernel algorithmic flops / bytes), data (the inputs)}."""
    rows = {}
    # time-branch decoder: the four UNetDecoderBlock levels at the config-4 lengths of a padded
    # chunk (344064 samples -> 86016 / 21504 / 5376 / 1344), with synthetic inputs and skips of
    # those shapes
    dec = decoder_setup(nn, dev)

    def f6():
        y = dec["x"]
        for blk, sk, out in zip(dec["blocks"], dec["skips"], dec["outs"]):
            blk.forward(y, sk, out, stream)
            y = out
    rows["6_time_decoder_b1"] = {"fn": f6, "flops": dec["flops"], "work": dec["work"],
                                 "data": dec}
    # frequency branch: the four 2-D encoder levels and the four decoder levels of the
    # reference's HTDemucs at one chunk's spectrogram (synthetic inputs and skips)
    fenc, fdec = freq_setup(nn, dev)

    def f7():
        y = fenc["x"]
        for blk, out in zip(fenc["blocks"], fenc["outs"]):
            blk.forward(y, out, stream)
            y = out

    def f8():
        y = fdec["x"]
        for blk, sk, out in zip(fdec["blocks"], fdec["skips"], fdec["outs"]):
            blk.forward(y, sk, out, stream)
            y = out
    rows["7_freq_encoder_b1"] = {"fn": f7, "flops": fenc["flops"], "work": fenc["work"],
                                 "data": fenc}
    rows["8_freq_decoder_b1"] = {"fn": f8, "flops": fdec["flops"], "work": fdec["work"],
                                 "data": fdec}
    # STFT / iSTFT of one stereo 7.8 s chunk at HTDemucs' nfft 4096 / hop 1024 (bin-major
    # spectrogram, as the frequency branch consumes it); bytes = signal read + spectra written
    # (forward), spectra read + signal written (inverse)
    xs = np.random.default_rng(1008).uniform(-1, 1, (2, 343980)).astype(np.float32)
    plan = nn.STFT(dev, 4096, 1024, "hann")
    xst = nn.Tensor.from_numpy(dev, xs)
    nf = plan.frame_count(343980)
    re9, im9 = nn.Tensor(dev, (2, 2049, nf)), nn.Tensor(dev, (2, 2049, nf))
    y9 = nn.Tensor(dev, (2, plan.output_length(nf)))
    from metalaudio_amd._lib import check as check9, lib as lib9

    def fwd():
        check9(lib9().mnn_stft_forward(plan.handle, xst.handle, re9.handle, im9.handle, 1, 1,
                                       stream.handle))

    def inv():
        check9(lib9().mnn_stft_inverse(plan.handle, re9.handle, im9.handle, 1, 1, 1e-10,
                                       y9.handle, stream.handle))
    spec_b = 2 * nf * 2049 * 8.0
    b9 = 4.0 * xs.size + spec_b
    rows["9_stft_b1"] = {"fn": fwd, "byts": b9, "floor": (4.0 * xs.size, spec_b),
                         "work": {"stft_forward_f32": (0, b9)}, "data": xs,
                         "keep": (plan, xst, re9, im9)}
    frames_b = 4.0 * 2 * nf * 4096
    sig_b = 4.0 * 2 * plan.output_length(nf)
    # algorithmic bytes of the inverse: the spectra read, the signal written (the frames the
    # first of its two kernels writes and the second reads are this build's intermediate)
    rows["10_istft_b1"] = {"fn": inv, "byts": spec_b + sig_b, "floor": (spec_b, sig_b),
                           "work": {"istft_frames_f32": (0, spec_b + frames_b),
                                    "istft_overlap_add_f32": (0, frames_b + sig_b)},
                           "keep": (plan, y9)}
    return rows


def profile_rows(nn, dev, stream, path):
    """Profiling mode of rows 6-10: a warm-up call of each row, then one call each on one stream
    (kernel timing on: every launch in host order) with the library's launch log on. Writes the
    log, each launch name prefixed with its row ("8_freq_decoder_b1:convt2d_f32_mfma ..."), to
    path, and the rows' per-kernel algorithmic work under the same prefixed names to
    path.work.json, for metalaudio_amd.profsummary pmc."""
    import ctypes
    from metalaudio_amd._lib import lib
    rows = next_rows(nn, dev, stream)
    for r in rows.values():
        r["fn"]()
    stream.sync()
    dev.set_kernel_timing(True)
    lines, work = [], {}
    for name, r in rows.items():
        lib().mnn_debug_set_launch_log(dev.handle, 1)
        r["fn"]()
        stream.sync()
        lib().mnn_debug_set_launch_log(dev.handle, 0)
        need = ctypes.c_size_t()
        lib().mnn_debug_launch_log(dev.handle, None, 0, ctypes.byref(need))
        buf = ctypes.create_string_buffer(need.value)
        rc = lib().mnn_debug_launch_log(dev.handle, buf, need.value, ctypes.byref(need))
        if rc != 0:
            log(f"launch log: status {rc}")
            sys.exit(1)
        lines += [f"{name}:{line}" for line in buf.value.decode().splitlines()]
        work.update({f"{name}:{k}": [float(v[0]), float(v[1])] for k, v in r["work"].items()})
    dev.set_kernel_timing(False)
    Path(path).parent.mkdir(parents=True, exist_ok=True)
    Path(path).write_text("\n".join(lines) + "\n")
    Path(path).with_suffix(".work.json").write_text(json.dumps(work))
    log(f"profile rows: {len(lines)} launches logged to {path}")


def config_table(nn, W, dev, stream, m, cpu=True):
    """GPU ms, achieved rate and roofline fraction of each BASELINE configuration, with the fp32
    oracle's CPU time on the host beside it (the oracle is only the CPU baseline here). gpu_ms:
    median over 50 event-timed samples after 5 warm-up calls (time_gpu); `kernels`: the row's
    per-kernel times from a kernel-timing pass; `floor`: the measured floor of a bandwidth-bound
    row's traffic (Floors)."""
    if cpu:
        import oracle
    out = {}

    floors = Floors(nn, dev, stream)

    def row(name, gpu_ms, flops=None, byts=None, prec="f32", cpu_ms=None, kernels=None,
            floor=None):
        r = {"gpu_ms": round(gpu_ms, 4), "calls_per_sample": getattr(time_gpu, "calls", 1)}
        if floor is not None:
            r["floor"] = floors.of(floor[0], floor[1], gpu_ms)
        if flops:
            r["tflops"] = round(flops / gpu_ms / 1e9, 2)
            r["mfma_frac"] = round(flops / (gpu_ms * 1e-3) / PEAK[prec], 4)
        if byts:
            r["gbps"] = round(byts / gpu_ms / 1e6, 1)
            r["hbm_frac"] = round(byts / (gpu_ms * 1e-3) / PEAK["hbm"], 4)
        if cpu_ms is not None:
            r["cpu_ms"] = round(cpu_ms, 2)
        if kernels is not None:
            r["kernels"] = kernels
        out[name] = r

    # config 1: Conv1D 2->48 k8 s4 -> GroupNorm(1) -> GELU (HBM-bound; bytes = x + y)
    c1 = W.config1()
    # as the reference composes it: Sequential [Conv1D, GroupNorm, GELU] (run as one fused
    # launch: each workgroup keeps its conv tile in registers, the workgroups exchange their
    # GroupNorm statistics partials, and each writes its normalised tile)
    conv = nn.Conv1D(dev, 2, 48, 8, stride=4, padding=0, input_length=44100)
    conv.load_weights(c1["conv_w"], c1["conv_b"])
    gn = nn.GroupNorm(dev, 1, 48)
    gn.load_parameters(c1["gn_w"], c1["gn_b"])
    gelu1 = nn.GELU(dev, [1, 48, 11024])
    seq1 = nn.Sequential(dev)
    for layer in (conv, gn, gelu1):
        seq1.add_unchecked(layer)
    seq1.build()
    x1 = nn.Tensor.from_numpy(dev, c1["x"])

    def f1():
        seq1.forward(x1, stream)
    cpu1 = time_cpu(lambda: oracle.gelu_layer(oracle.group_norm(oracle.conv1d(
        c1["x"], c1["conv_w"], c1["conv_b"], stride=4, dtype=np.float32), 1, c1["gn_w"],
        c1["gn_b"], dtype=np.float32), dtype=np.float32)) if cpu else None
    b1 = 4.0 * (2 * 44100 + 48 * 11024)
    row("1_conv_gn_gelu", time_gpu(f1, stream), flops=2.0 * 48 * 11024 * 16, byts=b1,
        cpu_ms=cpu1, floor=(4.0 * 2 * 44100, 4.0 * 48 * 11024), kernels=kernel_breakdown(dev, stream, f1, work={
            "conv_gn_oneshot_f32": (0, b1), "conv_gn_stats_f32": (0, 4.0 * 2 * 44100),
            "conv_gn_apply_f32": (0, b1)}))

    # config 2: Linear 512 -> 2048 on [2048, 512] + LayerNorm(2048), fp32 and bf16 operands
    c2 = W.config2()
    x2 = nn.Tensor.from_numpy(dev, c2["x"])
    y2 = nn.Tensor(dev, (2048, 2048))
    z2 = nn.Tensor(dev, (2048, 2048))
    ln = nn.LayerNorm(dev, 2048)
    ln.load_parameters(c2["ln_w"], c2["ln_b"])
    cpu2 = time_cpu(lambda: oracle.layer_norm(oracle.linear(c2["x"], c2["w"], c2["b"],
                                                            dtype=np.float32),
                                              c2["ln_w"], c2["ln_b"], dtype=np.float32)) \
        if cpu else None
    x2b = nn.Tensor.from_numpy(dev, c2["x"], dtype="bf16")  # bf16 X: 2 MB
    for prec in ("f32", "bf16"):
        lin = nn.Linear(dev, 512, 2048, precision=prec)
        lin.load_weights(c2["w"], c2["b"])
        xin = x2b if prec == "bf16" else x2

        def f2():
            lin.forward(xin, y2, stream)
            ln.forward(y2, z2, stream)
        # the Linear: fp32 on the matrix cores; bf16 (X and W bf16, Y fp32: 2 + 2 + 16 MB)
        # bound by HBM; the LayerNorm reads and writes 16 MB
        es = 2 if prec == "bf16" else 4
        g2 = (2.0 * 2048 * 2048 * 512, es * (2048 * 512 * 2) + 4.0 * 2048 * 2048)
        w2 = {f"gemm_{prec}_mfma_nk": g2, "layernorm_f32": (0, 8.0 * 2048 * 2048)}
        row(f"2_linear_ln_{prec}", time_gpu(f2, stream), flops=2.0 * 2048 * 2048 * 512,
            prec=prec, cpu_ms=cpu2 if prec == "f32" else None,
            kernels=kernel_breakdown(dev, stream, f2, work=w2, prec=prec))
        row(f"2_linear_{prec}", time_gpu(lambda: lin.forward(xin, y2, stream), stream),
            flops=g2[0], prec=prec, byts=g2[1],
            floor=(es * 2048 * 512 * 2, 4.0 * 2048 * 2048) if prec == "bf16" else None)
    # the LayerNorm over 2048 features alone (16 MB read, 16 MB written)
    row("2_layernorm_2048", time_gpu(lambda: ln.forward(y2, z2, stream), stream),
        byts=8.0 * 2048 * 2048, floor=(4.0 * 2048 * 2048, 4.0 * 2048 * 2048))

    # config 3: pre-norm MHSA + FFN layer, S 2048, E 512
    c3 = W.config3()
    tl = nn.TransformerLayer(dev, c3["embed"], c3["heads"], c3["ffn"])
    tl.load_state(c3["params"])
    x3 = nn.Tensor.from_numpy(dev, c3["x"])
    y3 = nn.Tensor(dev, x3.shape)
    cpu3 = time_cpu(lambda: oracle.transformer_layer(c3["x"], c3["params"], c3["heads"],
                                                     dtype=np.float32)) if cpu else None
    S, E = 2048, 512
    f3 = 2.0 * S * E * 3 * E + 4.0 * S * S * E + 2.0 * S * E * E + 4.0 * S * E * 2048
    row("3_transformer_layer", time_gpu(lambda: tl.forward(x3, y3, stream), stream),
        flops=f3, cpu_ms=cpu3)

    # configs 4 and 5 (the headline pair)
    enc = encoder_work()
    f4 = sum(v[0] for v in enc.values())
    row("4_encoder_b1", time_gpu(lambda: m["seq"].forward(m["chunks"][0], stream), stream),
        flops=f4)
    f5 = sum(v[0] for v in transformer_work(W.T5_BATCH).values())
    row("5_transformer_b4", time_gpu(lambda: run_transformer(m, stream), stream), flops=f5)
    nr = next_rows(nn, dev, stream)
    if cpu:
        from oracle import dsp as odsp  # CPU baseline only
    dec, fenc, fdec = nr["6_time_decoder_b1"]["data"], nr["7_freq_encoder_b1"]["data"], \
        nr["8_freq_decoder_b1"]["data"]
    xs = nr["9_stft_b1"]["data"]
    cpus = {}
    if cpu:
        cpus["6_time_decoder_b1"] = time_cpu(lambda: decoder_oracle(oracle, dec), max_reps=1)
        cpus["7_freq_encoder_b1"] = time_cpu(lambda: freq_encoder_oracle(oracle, fenc),
                                             max_reps=1)
        cpus["8_freq_decoder_b1"] = time_cpu(lambda: freq_decoder_oracle(oracle, fdec),
                                             max_reps=1)
        cpus["9_stft_b1"] = time_cpu(lambda: odsp.stft(xs, 4096, 1024, dtype=np.float32))
        X9 = odsp.stft(xs, 4096, 1024)
        cpus["10_istft_b1"] = time_cpu(lambda: odsp.istft(X9, 4096, 1024, dtype=np.float32))
    for name, r in nr.items():
        row(name, time_gpu(r["fn"], stream), flops=r.get("flops"), byts=r.get("byts"),
            cpu_ms=cpus.get(name), floor=r.get("floor"),
            kernels=kernel_breakdown(dev, stream, r["fn"], work=r["work"]))
    # long-audio driver: 60 s of stereo audio through the reference's default time-domain
    # HTDemucs (5 levels 48..768, k 8, s 4, 4 stems) in the guide's 30 s segments with 2 s
    # overlap (HTDEMUCS_GUIDE.md:170-191); synthetic weights and audio
    if cpu:
        from oracle import separate as osep  # CPU baseline only
    r11, cfg11, P11 = long_audio_setup()
    sep = nn.Separator(dev)
    sep.load_state(P11)
    n11 = 44100 * 60
    x11 = nn.Tensor.from_numpy(dev, r11.uniform(-1, 1, 2 * n11).astype(np.float32))
    o11 = nn.Tensor(dev, (4, 2 * n11))
    from metalaudio_amd._lib import check as check11, lib as lib11

    def f11():
        check11(lib11().mnn_separator_separate_long(sep.handle, x11.handle, o11.handle,
                                                    44100 * 30, 44100 * 2, stream.handle))
    seg_cpu = r11.uniform(-1, 1, 2 * 44100 * 10).astype(np.float32)
    cpu11 = time_cpu(lambda: osep.separate_time(seg_cpu, P11, cfg11, dtype=np.float32),
                     max_reps=1) * 6.0 if cpu else None
    g11 = time_gpu(f11, stream)
    row("11_long_audio_60s", g11, cpu_ms=cpu11, kernels=kernel_breakdown(dev, stream, f11, reps=3))
    out["11_long_audio_60s"]["x_realtime"] = round(60e3 / g11, 1)
    t5 = nn.Tensor.from_numpy(dev, m["c5"]["time"][:1])
    q5 = nn.Tensor.from_numpy(dev, m["c5"]["freq"][:1])
    to5, fo5 = nn.Tensor(dev, t5.shape), nn.Tensor(dev, q5.shape)
    row("5_transformer_b1", time_gpu(lambda: m["ct"].forward_cross(t5, q5, to5, fo5, stream),
                                     stream, 5), flops=f5 / W.T5_BATCH)
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--precision", choices=["f32", "bf16"], default="f32")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=40.0,
                    help="seconds of timed CPU-baseline runs at most")
    ap.add_argument("--no-configs", action="store_true", help="skip the per-configuration table")
    ap.add_argument("--profile-step", metavar="LOG",
                    help="profiling mode: after the warm-up, run ONE step on one stream with the "
                         "library's launch log on, write the log (one line per launch: name, "
                         "grid, block) to LOG and exit; metalaudio_amd.profsummary pmc attributes "
                         "a rocprofv3 run of this mode to the kernel names")
    ap.add_argument("--profile-rows", metavar="LOG",
                    help="profiling mode: run rows 6-10 of the configuration table once each "
                         "(after a warm-up call) on one stream with the launch log on, write the "
                         "log (names prefixed with the row) to LOG and exit; for "
                         "metalaudio_amd.profsummary pmc")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this path runs on a single MI355X with no "
              "sharding or collectives (--gpus 1).", file=sys.stderr)
        sys.exit(2)

    from metalaudio_amd import nn
    from metalaudio_amd import workloads as W

    dev = nn.AudioDevice(0)
    stream = nn.Stream(dev)
    if args.profile_rows:
        profile_rows(nn, dev, stream, args.profile_rows)
        return
    log(f"device {dev.name}; building models ({args.precision})")
    m = build_models(nn, W, dev, args.precision)

    def step():
        run_encoder(m, stream)
        run_transformer(m, stream)

    log(f"warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    stream.sync()

    if args.profile_step:
        import ctypes
        from metalaudio_amd._lib import lib
        # kernel timing on: every launch goes to the caller's stream, in host order
        dev.set_kernel_timing(True)
        lib().mnn_debug_set_launch_log(dev.handle, 1)
        step()
        stream.sync()
        lib().mnn_debug_set_launch_log(dev.handle, 0)
        dev.set_kernel_timing(False)
        need = ctypes.c_size_t()
        lib().mnn_debug_launch_log(dev.handle, None, 0, ctypes.byref(need))
        buf = ctypes.create_string_buffer(need.value)
        rc = lib().mnn_debug_launch_log(dev.handle, buf, need.value, ctypes.byref(need))
        if rc != 0:
            log(f"launch log: status {rc}")
            sys.exit(1)
        text = buf.value.decode()
        Path(args.profile_step).parent.mkdir(parents=True, exist_ok=True)
        Path(args.profile_step).write_text(text)
        work = encoder_work("enc_conv_reduce_gn" in text, "enc_l1_oneshot" in text)
        work = {k: [v[0] * 4, v[1] * 4] for k, v in work.items()}
        work.update(transformer_work(W.T5_BATCH))
        Path(args.profile_step).with_suffix(".work.json").write_text(json.dumps(work))
        log(f"profile step: {len(text.splitlines())} launches logged to {args.profile_step}")
        return

    markers = Markers()
    # timed region: wall clock around exactly K steps (no per-launch events)
    log(f"timing {args.steps} steps")
    markers.push("bench:timed")
    ms_step = timed(step, stream, args.steps)
    markers.pop()

    # kernel-timing pass: K more steps with a HIP event pair around every launch, recorded on the
    # stream the kernel runs on; gives each family's average launch duration (the events add
    # gaps between launches, which is why the headline above is timed without them)
    dev.reset_kernel_timing()
    dev.set_kernel_timing(True)
    markers.push("bench:kernel_timing")
    ms_step_events = timed(step, stream, args.steps)
    markers.pop()
    dev.set_kernel_timing(False)
    fams = ["attn_fwd", "gemm_f32_mfma_nk", "gemm_f32_mfma_kn", "gemm_f32_mfma_conv",
            "gemm_f32_simple", "conv1d_direct", "layernorm", "ln_row_parts_f32", "ln_fold_f32",
            "gn_stats", "gn_finalize", "gn_apply", "copy_bytes", "glu_f32", "gelu_f32"]
    # per level, e.g. enc_conv_f32[c96]; the forms that ran decide the accounting
    enc_names = sorted(set(encoder_work(True)) | set(encoder_work(False)))
    ktime = {}
    for f in fams + enc_names:
        n, ms = dev.kernel_timing(f)
        if n:
            ktime[f] = (n, ms)
    ew = encoder_work(any(k.startswith("enc_conv_reduce_gn") for k in ktime),
                      any(k.startswith("enc_l1_oneshot") for k in ktime))
    enc_kernels = list(ew)
    log("kernel ms/step: " + ", ".join(f"{k}={v[1] / args.steps:.3f} ({v[0] // args.steps})"
                                        for k, v in ktime.items()))

    # breakdown (no events): encoder alone and transformer alone
    t_enc = timed(lambda: run_encoder(m, stream), stream, max(2, args.steps // 2)) / 4
    t_tr = timed(lambda: run_transformer(m, stream), stream, max(2, args.steps // 2))
    log(f"ms/step {ms_step:.3f}; encoder {t_enc:.3f} ms/chunk; transformer b4 {t_tr:.3f} ms")

    # roofline of the dominant family
    work = {k: [v[0] * 4, v[1] * 4] for k, v in ew.items()}  # 4 chunks per step
    for k, v in transformer_work(W.T5_BATCH).items():
        work[k] = v
    fam_key = {"attn_fwd": "attn_fwd_f32"}
    rows = {}
    for f, (n, ms) in ktime.items():
        wk = work.get(fam_key.get(f, f))
        if not wk:
            continue
        t = ms / 1e3 / args.steps  # seconds per step
        flops, byts = wk
        bound = "mfma" if flops > 0 and flops / max(byts, 1) > 20 else "hbm"
        if bound == "mfma":
            ach = flops / t
            peak = PEAK["bf16" if args.precision == "bf16" else "f32"]
            rows[f] = {"bound": "mfma", "achieved": round(ach / 1e12, 2),
                       "peak": round(peak / 1e12, 1), "unit": "TFLOP/s",
                       "frac": round(ach / peak, 4), "ms_per_step": round(t * 1e3, 3),
                       "launches_per_step": n // args.steps}
        else:
            ach = byts / t
            rows[f] = {"bound": "hbm", "achieved": round(ach / 1e9, 1), "peak": 8000.0,
                       "unit": "GB/s", "frac": round(ach / PEAK["hbm"], 4),
                       "ms_per_step": round(t * 1e3, 3), "launches_per_step": n // args.steps}
    # the encoder as a whole (all its kernels, one chunk's algorithmic flops)
    enc_ms = sum(ktime[k][1] for k in enc_kernels if k in ktime) / args.steps
    if enc_ms > 0:
        ef = 4 * sum(ew[k][0] for k in enc_kernels)  # 4 chunks per step
        rows["encoder_all_levels"] = {
            "bound": "mfma", "achieved": round(ef / (enc_ms / 1e3) / 1e12, 2), "peak": 157.3,
            "unit": "TFLOP/s", "frac": round(ef / (enc_ms / 1e3) / PEAK["f32"], 4),
            "ms_per_step": round(enc_ms, 3),
            "launches_per_step": sum(ktime[k][0] for k in enc_kernels if k in ktime) // args.steps}
    dom = max((k for k in ktime if k in rows), key=lambda k: ktime[k][1])
    roof = dict(rows.get(dom, {}))
    roof["kernel"] = dom
    traffic = None
    tf = ROOT / "profiles" / "traffic.json"
    if tf.exists():
        try:
            traffic = json.loads(tf.read_text()).get(dom)
        except Exception:
            traffic = None
    roof["traffic"] = traffic
    roof["avg_launch_us"] = round(ktime[dom][1] / ktime[dom][0] * 1e3, 2)

    configs = None
    if not args.no_configs:
        log("per-configuration table")
        configs = config_table(nn, W, dev, stream, m, cpu=not args.no_cpu_baseline)

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        cpu = cpu_baseline(m, budget_s=args.cpu_budget)

    out = {
        "metric": METRIC,
        "value": round(ms_step / 4, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.precision,
        "data": "synthetic (seeded PCG64 inputs and weights of the BASELINE config shapes)",
        "config": {
            "workload": "config 4 (4-level time encoder, 2x343980 samples, batch 1) on 4 chunks "
                        "+ config 5 (5-layer cross transformer, time 1344 / freq 2688 tokens, "
                        "E 384, H 8, FFN 1536) at batch 4; value = step / 4 chunks",
            "chunks_per_step": 4,
            "encoder_ms_per_chunk": round(t_enc, 4),
            "ms_per_step_with_kernel_events": round(ms_step_events, 4),
            "transformer_b4_ms": round(t_tr, 4),
        },
        "roofline": roof,
        "kernels": rows,
        "configs": configs,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
