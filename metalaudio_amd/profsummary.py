"""Summaries of rocprofv3 output for the profiles/ folder.

Subcommands:
  trace DIR --cmd "..." [--out FILE]
      per-kernel table (calls, average / min / total microseconds, share) from the
      *kernel_trace.csv of a `rocprofv3 --kernel-trace` run;
  stats DIR --cmd "..." [--out FILE]
      the *kernel_stats.csv of a `rocprofv3 --stats` run as a table (calls, average / min / max /
      total microseconds, share);
  copy --mib N
      a plain device copy of N MiB (torch), the calibration run for the HBM counters;
  pmc --log LOG --trace DIR --passes DIR [DIR ...] --fetch DIR --write DIR --copy-fetch DIR
      --copy-write DIR --copy-mib N --cmd "..." [--cmd "..."] [--out FILE] [--traffic-out FILE]
      per-family table of one bench step (`bench.py --profile-step LOG`): durations from a kernel
      trace, MFMA busy / VALU per MFMA / wait / LDS bank conflicts from SQ counter passes, HBM
      bytes from FETCH_SIZE / WRITE_SIZE against the algorithmic bytes; dispatches are attributed
      to the library's launch names through the launch log;
  traffic --fetch DIR --write DIR --copy-fetch DIR --copy-write DIR --copy-mib N [--out FILE]
      HBM bytes per dispatch of each kernel family from two `rocprofv3 --pmc` runs (FETCH_SIZE,
      then WRITE_SIZE, KiB per dispatch), each scaled by the factor that makes the same counter
      read the known size of the copy run; written as JSON {family: bytes per launch}.

Kernel families are the names the library's kernel timing uses (bench.py reports them).
"""
from __future__ import annotations

import argparse
import collections
import csv
import glob
import json
import re
import statistics
import subprocess
import sys
from pathlib import Path

# kernel symbol (substring) -> kernel-timing family of the library
FAMILIES = [
    ("attn_fwd_f32_kernel", "attn_fwd"),
    ("attn_generic_kernel", "attn_fwd"),
    ("attn_combine_kernel", "attn_combine_f32"),
    ("stft_forward_sk_kernel", "stft_forward_f32"),
    ("stft_inverse_sk_kernel", "istft_frames_f32"),
    ("enc_l1_stats_kernel", "enc_l1_stats_f32"),
    ("enc_l1_fused_kernel", "enc_l1_fused_f32"),
    ("enc_l1_oneshot_kernel", "enc_l1_oneshot_f32"),
    ("enc_reduce_gn_t_kernel", "enc_conv_reduce_gn_f32"),
    ("floor_empty_kernel", "floor_empty"),
    ("floor_stream_kernel", "floor_stream"),
    ("conv_gn_oneshot_kernel", "conv_gn_oneshot_f32"),
    ("conv_gn_stats_kernel", "conv_gn_stats_f32"),
    ("zero_u32_kernel", "zero_u32"),
    ("conv_gn_apply_kernel", "conv_gn_apply_f32"),
    ("conv1d_direct", "conv1d_direct_f32"),
    ("gn_apply_parts_kernel", "gn_apply_parts"),
    ("gemm_nk_lds_kernel", "gemm_f32_mfma_nk"),
    ("enc_conv_reduce_kernel", "enc_conv_reduce_f32"),
    ("enc_conv_kernel", "enc_conv_f32"),
    ("enc_gn_gelu_t_kernel", "enc_gn_gelu_t_f32"),
    ("convt_pack_kernel", "convt_pack_f32"),
    ("convt_direct_kernel", "convt_direct_f32"),
    ("convt_small_kernel", "convt_small_f32"),
    ("convt_reduce_kernel", "convt_reduce_f32"),
    ("conv2d_unfold_kernel", "conv2d_unfold_f32"),
    ("conv2d_unfold_tiled_kernel", "conv2d_unfold_f32"),
    ("conv2d_small_kernel", "conv2d_small_f32"),
    ("conv2d_split_reduce_kernel", "conv2d_split_reduce_f32"),
    ("conv2d_split_reduce_gn_kernel", "conv2d_split_reduce_f32"),
    ("conv2d_igemm_kernel", "conv2d_igemm_f32"),
    ("convt2d_gather_fixed_kernel", "convt2d_gather_f32"),
    ("convt2d_small_kernel", "convt2d_small_f32"),
    ("conv2d_direct_kernel", "conv2d_direct_f32"),
    ("convt2d_gather_kernel", "convt2d_gather_f32"),
    ("convt2d_gather_phase_kernel", "convt2d_gather_f32"),
    ("convt2d_direct_kernel", "convt2d_direct_f32"),
    ("stft_forward_kernel", "stft_forward_f32"),
    ("stft_inverse_kernel", "istft_frames_f32"),
    ("stft_overlap_add_kernel", "istft_overlap_add_f32"),
    ("deinterleave_pad_kernel", "deinterleave_pad_f32"),
    ("crossfade_store_kernel", "crossfade_store_f32"),
    ("gn_stats_partial_kernel", "gn_stats"),
    ("gn_finalize_kernel", "gn_finalize"),
    ("gn_apply_kernel", "gn_apply"),
    ("gemm_f32_mfma_kernel", "gemm_f32_mfma"),
    ("layernorm", "layernorm"),
    ("ln_row_parts_kernel", "ln_row_parts_f32"),
    ("ln_fold_kernel", "ln_fold_f32"),
    ("copy_kernel", "copy_bytes"),
]


def _demangle(names):
    try:
        out = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True,
                             check=True).stdout.splitlines()
        return dict(zip(names, out))
    except (OSError, subprocess.CalledProcessError):
        return {n: n for n in names}


def _short(name: str) -> str:
    name = name.replace("(anonymous namespace)::", "")
    name = re.sub(r"\(.*", "", name)
    return name.split("::")[-1] if "<" not in name else name[name.rfind("::", 0, name.find("<")) + 2:]


def _family(name: str) -> str:
    if "gemm_nk_lds_kernel" in name:
        # template arguments: WMW, WNW, WM, WN, S, EPI[, BF]
        args = name[name.find("<") + 1:name.rfind(">")].replace(" ", "").split(",")
        epi = args[5] if len(args) > 5 else ""
        if len(args) > 6 and args[6] == "true":
            return "gemm_bf16_mfma_nk"
        if epi == "1":
            return "enc_rewrite_f32"  # the GLU epilogue instantiation
        if epi == "2":
            return "convt_f32_mfma"  # the transposed-conv epilogue instantiation
    for key, fam in FAMILIES:
        if key in name:
            return fam
    return name


def _csvs(d: str, suffix: str):
    return glob.glob(str(Path(d) / "**" / f"*{suffix}"), recursive=True)


def _range(d: str, name: str):
    """(start, end) of the first roctx range `name` in a --marker-trace run."""
    for p in _csvs(d, "marker_api_trace.csv"):
        for r in csv.DictReader(open(p)):
            msg = r.get("Message") or r.get("Marker_Message") or r.get("Function", "")
            if msg == name:
                return int(r["Start_Timestamp"]), int(r["End_Timestamp"])
    raise SystemExit(f"range {name!r} not found in the marker trace under {d}")


def trace(args) -> str:
    rows = []
    for p in _csvs(args.dir, "kernel_trace.csv"):
        rows += list(csv.DictReader(open(p)))
    if args.range:
        t0, t1 = _range(args.dir, args.range)
        rows = [r for r in rows if int(r["Start_Timestamp"]) >= t0 and int(r["End_Timestamp"]) <= t1]
    dm = _demangle(sorted({r["Kernel_Name"] for r in rows}))
    by = collections.defaultdict(list)
    for r in rows:
        k = _short(dm[r["Kernel_Name"]])
        by[k].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    total = sum(sum(v) for v in by.values()) or 1.0
    scope = (f"dispatches inside the roctx range `{args.range}`" if args.range
             else "dispatches over the whole run")
    lines = [f"# {args.title}", "", "Command (repo root, GPU box):", "", "```", args.cmd, "```", "",
             f"Per kernel instantiation: {scope}, duration from the kernel trace.", "",
             "| kernel | family | calls | avg us | min us | total us | % |",
             "|---|---|---|---|---|---|---|"]
    for k, v in sorted(by.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| `{k}` | {_family(k)} | {len(v)} | {statistics.mean(v):.1f} | "
                     f"{min(v):.1f} | {sum(v):.0f} | {100 * sum(v) / total:.1f} |")
    fam = collections.defaultdict(list)
    for k, v in by.items():
        fam[_family(k)] += v
    lines += ["", "Per family:", "", "| family | calls | avg us | total us |", "|---|---|---|---|"]
    for f, v in sorted(fam.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| {f} | {len(v)} | {statistics.mean(v):.1f} | {sum(v):.0f} |")
    return "\n".join(lines) + "\n"


def stats(args) -> str:
    rows = []
    for p in _csvs(args.dir, "kernel_stats.csv"):
        rows += list(csv.DictReader(open(p)))
    dm = _demangle(sorted({r["Name"] for r in rows}))
    lines = [f"# {args.title}", "", "Command (repo root, GPU box):", "", "```", args.cmd, "```", "",
             "`*_kernel_stats.csv` of the run, durations in microseconds.", "",
             "| kernel | family | calls | avg us | min us | max us | total us | % |",
             "|---|---|---|---|---|---|---|---|"]
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    for r in rows:
        k = _short(dm[r["Name"]])
        lines.append(f"| `{k}` | {_family(k)} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                     f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | "
                     f"{float(r['TotalDurationNs']) / 1e3:.0f} | {float(r['Percentage']):.1f} |")
    return "\n".join(lines) + "\n"


def floors(args) -> str:
    """Measured floors of a configuration-table run (bench.py's Floors): the empty launch and
    each size of the streaming kernel (its grid follows max(read, write) bytes: 64 bytes per
    thread), beside the bandwidth-bound rows' own kernels from the same trace."""
    rows = []
    for p in _csvs(args.dir, "kernel_trace.csv"):
        rows += list(csv.DictReader(open(p)))
    dm = _demangle(sorted({r["Kernel_Name"] for r in rows}))
    fl = collections.defaultdict(list)
    rk = collections.defaultdict(list)
    watch = ("conv_gn_oneshot_f32", "layernorm", "gemm_bf16_mfma_nk", "stft_forward_f32",
             "istft_frames_f32", "istft_overlap_add_f32")
    for r in rows:
        k = _short(dm[r["Kernel_Name"]])
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        threads = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        fam = _family(k)
        if fam in ("floor_empty", "floor_stream"):
            fl[(fam, threads if fam == "floor_stream" else 0)].append(us)
        elif fam in watch:
            rk[fam].append(us)
    med = statistics.median
    lines = [f"# {args.title}", "", "Command (repo root, GPU box):", "", "```", args.cmd, "```", "",
             "Kernel-trace durations (microseconds) of the floor kernels that bench.py's "
             "configuration table launches beside its bandwidth-bound rows: an empty launch, and one "
             "streaming pass (`floor_stream_kernel`, 16-byte loads and stores) per traffic size; "
             "the pass's grid follows max(read, write) bytes, 64 bytes per thread, so rows with the "
             "same larger side share a line (the LayerNorm's 16 + 16 MB and the bf16 Linear's 4 + 16 "
             "MB). The rows' own kernels from the same trace follow.", "",
             "| floor | max(read, write) MB | rows | calls | median us | min us |",
             "|---|---|---|---|---|---|"]
    rows_of = {2.1: "config 1 (0.35 MB read, 2.1 MB written)",
               10.9: "STFT (2.75 read, 10.9 written), iSTFT (10.9 read, 2.74 written)",
               16.8: "config-2 LayerNorm (16.8 + 16.8), bf16 Linear (4.2 + 16.8)"}
    for (fam, threads), v in sorted(fl.items()):
        mb = threads * 64 / 1e6
        near = min(rows_of, key=lambda m: abs(m - mb)) if fam == "floor_stream" else None
        label = rows_of[near] if near is not None and abs(near - mb) < 0.5 else ""
        lines.append(f"| {'empty launch' if fam == 'floor_empty' else 'streaming pass'} | "
                     f"{'-' if fam == 'floor_empty' else f'{mb:.1f}'} | {label} | {len(v)} | "
                     f"{med(v):.2f} | {min(v):.2f} |")
    lines += ["", "| row kernel (same trace) | calls | median us | min us |", "|---|---|---|---|"]
    for fam in watch:
        if rk.get(fam):
            lines.append(f"| {fam} | {len(rk[fam])} | {med(rk[fam]):.2f} | {min(rk[fam]):.2f} |")
    return "\n".join(lines) + "\n"


def _counter_per_dispatch(d: str, counter: str):
    """{kernel name: [counter value per dispatch]} from a --pmc run."""
    per = collections.defaultdict(float)
    names = {}
    for p in _csvs(d, "counter_collection.csv"):
        for r in csv.DictReader(open(p)):
            if r["Counter_Name"] != counter:
                continue
            key = (p, r["Dispatch_Id"])
            per[key] += float(r["Counter_Value"])  # summed over XCDs / instances
            names[key] = r["Kernel_Name"]
    out = collections.defaultdict(list)
    for key, v in per.items():
        out[names[key]].append(v)
    return out


def traffic(args) -> dict:
    copy_bytes = args.copy_mib * 1024 * 1024
    res = {}
    for counter, d, cd in (("FETCH_SIZE", args.fetch, args.copy_fetch),
                           ("WRITE_SIZE", args.write, args.copy_write)):
        cal = _counter_per_dispatch(cd, counter)
        big = max((max(v) for v in cal.values()), default=0.0)  # the copy is the largest dispatch
        factor = copy_bytes / (big * 1024.0) if big > 0 else 1.0
        res[counter] = {"factor": factor}
        per = _counter_per_dispatch(d, counter)
        dm = _demangle(sorted(per))
        fam = collections.defaultdict(list)
        for k, v in per.items():
            fam[_family(_short(dm[k]))] += v
        for f, v in fam.items():
            res[counter][f] = statistics.mean(v) * 1024.0 * factor
    out = {"_note": "HBM bytes per dispatch: FETCH_SIZE + WRITE_SIZE (KiB) x copy-calibrated factor",
           "_factors": {"FETCH_SIZE": res["FETCH_SIZE"]["factor"],
                        "WRITE_SIZE": res["WRITE_SIZE"]["factor"]}}
    for f in set(res["FETCH_SIZE"]) | set(res["WRITE_SIZE"]):
        if f == "factor":
            continue
        out[f] = round(res["FETCH_SIZE"].get(f, 0.0) + res["WRITE_SIZE"].get(f, 0.0))
    return out


# ------------------------------------------------------------------ per-family counter table
CLOCK_HZ = 2.4e9   # MI355X peak engine clock: cycles -> seconds for the MFMA busy fraction
SIMDS = 1024       # 256 CUs x 4 SIMDs
PEAK = {"hbm": 8.0e12, "f32": 157.3e12}


def _dispatches(d: str):
    """Library dispatches of a rocprofv3 run in dispatch order: list of dicts with the kernel
    name, total threads, workgroup size, start / end and {counter: value} (summed over
    instances). Runtime-internal kernels (__amd_rocclr_*) are left out."""
    disp = {}
    for p in _csvs(d, "kernel_trace.csv"):
        for r in csv.DictReader(open(p)):
            if r["Kernel_Name"].startswith("__amd"):
                continue
            threads = (int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"]))
            disp[(p, int(r["Dispatch_Id"]))] = {
                "name": r["Kernel_Name"], "threads": threads,
                "wg": int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) *
                int(r["Workgroup_Size_Z"]),
                "t": (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3, "c": {}}
    for p in _csvs(d, "counter_collection.csv"):
        for r in csv.DictReader(open(p)):
            if r["Kernel_Name"].startswith("__amd"):
                continue
            key = (p, int(r["Dispatch_Id"]))
            e = disp.setdefault(key, {"name": r["Kernel_Name"], "threads": int(r["Grid_Size"]),
                                      "wg": int(r["Workgroup_Size"]), "t": None, "c": {}})
            e["c"][r["Counter_Name"]] = e["c"].get(r["Counter_Name"], 0.0) + \
                float(r["Counter_Value"])
    return [disp[k] for k in sorted(disp)]


def _align(d: str, log):
    """The last len(log) dispatches of run d, checked launch by launch against the log's grid
    and workgroup sizes."""
    ds = _dispatches(d)
    if len(ds) < len(log):
        raise SystemExit(f"{d}: {len(ds)} dispatches, the launch log has {len(log)}")
    ds = ds[-len(log):]
    for i, (e, l) in enumerate(zip(ds, log)):
        if e["threads"] != l["threads"] or e["wg"] != l["wg"]:
            raise SystemExit(f"{d}: dispatch {i} ({e['name'][:60]}, {e['threads']} threads) does "
                             f"not match launch {l['name']} ({l['threads']} threads)")
    return ds


def _read_log(path: str):
    out = []
    for line in Path(path).read_text().splitlines():
        name, gx, gy, gz, bx = line.rsplit(" ", 4)
        out.append({"name": name, "threads": int(gx) * int(gy) * int(gz) * int(bx),
                    "wg": int(bx)})
    return out


def _work_key(name: str, work: dict):
    keys = [k for k in work if k in name]
    return max(keys, key=len) if keys else None


def pmc(args) -> str:
    log = _read_log(args.log)
    work = json.loads(Path(args.log).with_suffix(".work.json").read_text())
    trace = _align(args.trace, log)
    passes = [_align(d, log) for d in args.passes]
    fetch = _align(args.fetch, log)
    write = _align(args.write, log)
    fac = {}
    for counter, cd in (("FETCH_SIZE", args.copy_fetch), ("WRITE_SIZE", args.copy_write)):
        cal = _counter_per_dispatch(cd, counter)
        big = max((max(v) for v in cal.values()), default=0.0)
        fac[counter] = args.copy_mib * 1024 * 1024 / (big * 1024.0) if big > 0 else 1.0
    fam = collections.OrderedDict()
    for i, l in enumerate(log):
        key = _work_key(l["name"], work) or l["name"]
        f = fam.setdefault(key, {"n": 0, "t": 0.0, "c": collections.defaultdict(float),
                                 "hbm": 0.0, "names": set()})
        f["n"] += 1
        f["t"] += trace[i]["t"]
        f["names"].add(l["name"])
        for ps in passes:
            for c, v in ps[i]["c"].items():
                f["c"][c] += v
        f["hbm"] += (fetch[i]["c"].get("FETCH_SIZE", 0.0) * fac["FETCH_SIZE"] +
                     write[i]["c"].get("WRITE_SIZE", 0.0) * fac["WRITE_SIZE"]) * 1024.0
    lines = [f"# {args.title}", "", "Commands (repo root, GPU box):", "", "```"] + \
        args.cmd + ["```", "",
                    f"{args.scope} ({len(log)} launches, kernel timing on so that every launch "
                    "runs on one stream in host order), attributed to the library's launch names "
                    "by the launch log (grid and workgroup sizes checked dispatch by dispatch). "
                    f"{args.per}:", "",
                    "* `us`: summed kernel-trace duration; `frac`: algorithmic FLOP/s (MFMA-bound "
                    "rows) or bytes/s (HBM-bound rows) over the MI355X peak (157.3 TFLOP/s fp32, "
                    "8 TB/s);",
                    "* `MFMA busy`: SQ_VALU_MFMA_BUSY_CYCLES / (duration x 2.4 GHz x 1024 SIMDs); "
                    "`VALU/MFMA`: SQ_INSTS_VALU / SQ_INSTS_MFMA; `wait`: SQ_WAIT_INST_ANY / "
                    "SQ_WAVE_CYCLES (share of wave time waiting on an outstanding memory / LDS "
                    "result); `LDS confl.`: SQ_LDS_BANK_CONFLICT / SQ_INSTS_LDS;",
                    f"* `HBM MB`: FETCH_SIZE + WRITE_SIZE (KiB per dispatch) x the factor that makes "
                    f"the same counter read a {args.copy_mib} MiB copy's size (FETCH "
                    f"{fac['FETCH_SIZE']:.3f}, WRITE {fac['WRITE_SIZE']:.3f}); `alg MB`: the "
                    "algorithmic bytes bench.py prices the family with.", "",
                    "| family | launches | us | bound | frac | MFMA busy | VALU/MFMA | wait | "
                    "LDS confl. | HBM MB | alg MB | HBM/alg |",
                    "|---|---|---|---|---|---|---|---|---|---|---|---|"]
    traffic = {"_note": "HBM bytes per launch (FETCH_SIZE + WRITE_SIZE, copy-calibrated), one "
                        "bench step", "_factors": fac}
    for key, f in sorted(fam.items(), key=lambda kv: -kv[1]["t"]):
        c = f["c"]
        t = f["t"] * 1e-6
        flops, byts = work.get(key, [0.0, 0.0])
        mfma_bound = flops > 0 and flops / max(byts, 1.0) > 20
        if key in work and t > 0:
            frac = (flops / t / PEAK["f32"]) if mfma_bound else (byts / t / PEAK["hbm"])
            frac_s = f"{frac:.2f}"
        else:
            frac_s = "-"
        busy = c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (t * CLOCK_HZ * SIMDS) if t > 0 else 0
        vm = (c["SQ_INSTS_VALU"] / c["SQ_INSTS_MFMA"]) if c.get("SQ_INSTS_MFMA") else None
        wait = (c["SQ_WAIT_INST_ANY"] / c["SQ_WAVE_CYCLES"]) if c.get("SQ_WAVE_CYCLES") else None
        confl = (c["SQ_LDS_BANK_CONFLICT"] / c["SQ_INSTS_LDS"]) if c.get("SQ_INSTS_LDS") and \
            "SQ_LDS_BANK_CONFLICT" in c else None
        lines.append(
            f"| {key} | {f['n']} | {f['t']:.1f} | {'MFMA' if mfma_bound else 'HBM'} | {frac_s} | "
            f"{busy:.2f} | {'-' if vm is None else f'{vm:.1f}'} | "
            f"{'-' if wait is None else f'{wait:.2f}'} | "
            f"{'-' if confl is None else f'{confl:.2f}'} | {f['hbm'] / 1e6:.1f} | "
            f"{byts / 1e6:.1f} | {f['hbm'] / byts if byts else 0:.2f} |")
        traffic[key] = round(f["hbm"] / f["n"])
    if args.traffic_out:
        Path(args.traffic_out).write_text(json.dumps(traffic, indent=1, sort_keys=True) + "\n")
    return "\n".join(lines) + "\n"


def copy(args) -> None:
    import torch
    n = args.mib * 1024 * 1024 // 4
    src = torch.ones(n, device="cuda", dtype=torch.float32)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copied {args.mib} MiB x 3", flush=True)


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    sub = ap.add_subparsers(dest="cmd_name", required=True)
    t = sub.add_parser("trace")
    t.add_argument("dir")
    t.add_argument("--cmd", required=True)
    t.add_argument("--title", default="rocprofv3 kernel trace")
    t.add_argument("--range", help="only dispatches inside this roctx range")
    t.add_argument("--out")
    st = sub.add_parser("stats")
    st.add_argument("dir")
    st.add_argument("--cmd", required=True)
    st.add_argument("--title", default="rocprofv3 --stats")
    st.add_argument("--out")
    fo = sub.add_parser("floors")
    fo.add_argument("dir")
    fo.add_argument("--cmd", required=True)
    fo.add_argument("--title", default="measured floors of the configuration table")
    fo.add_argument("--out")
    c = sub.add_parser("copy")
    c.add_argument("--mib", type=int, default=1024)
    f = sub.add_parser("traffic")
    for k in ("fetch", "write", "copy_fetch", "copy_write"):
        f.add_argument("--" + k.replace("_", "-"), dest=k, required=True)
    f.add_argument("--copy-mib", type=int, required=True)
    f.add_argument("--out")
    q = sub.add_parser("pmc")
    q.add_argument("--log", required=True, help="launch log of bench.py --profile-step")
    q.add_argument("--trace", required=True, help="rocprofv3 --kernel-trace run of the same step")
    q.add_argument("--passes", nargs="+", required=True, help="rocprofv3 --pmc runs (SQ counters)")
    for k in ("fetch", "write", "copy_fetch", "copy_write"):
        q.add_argument("--" + k.replace("_", "-"), dest=k, required=True)
    q.add_argument("--copy-mib", type=int, required=True)
    q.add_argument("--cmd", action="append", required=True)
    q.add_argument("--title", default="per-family counters of one bench step")
    q.add_argument("--traffic-out")
    q.add_argument("--scope", default="One bench step", help="what the launch log covers")
    q.add_argument("--per", default="Per family and step", help="lead-in of the column list")
    q.add_argument("--out")
    a = ap.parse_args(argv)
    if a.cmd_name in ("trace", "stats", "floors"):
        text = trace(a) if a.cmd_name == "trace" else stats(a) if a.cmd_name == "stats" else floors(a)
        if a.out:
            Path(a.out).write_text(text)
        print(text)
    elif a.cmd_name == "copy":
        copy(a)
    elif a.cmd_name == "pmc":
        text = pmc(a)
        if a.out:
            Path(a.out).write_text(text)
        print(text)
    else:
        d = traffic(a)
        if a.out:
            Path(a.out).write_text(json.dumps(d, indent=1) + "\n")
        print(json.dumps(d, indent=1))


if __name__ == "__main__":
    main(sys.argv[1:])
