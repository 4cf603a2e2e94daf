"""Summaries of rocprofv3 output for the Q4 decode kernels.

    python -m measure.profiling stats <dir>
        per-kernel calls / average / min / max duration from a
        ``rocprofv3 --kernel-trace --stats`` output directory.
    python -m measure.profiling launches <dir>
        the same run's Q4 dispatches grouped by launch shape (grid, LDS).
    python -m measure.profiling counters <dir>
        mean per dispatch of every counter of a ``--pmc`` run, per Q4 kernel.
    python -m measure.profiling decode <dir>
        per-op medians of a decode-step run (bench.py --decode-step under
        ``--kernel-trace``), each launch named by its place in the step.
    python -m measure.profiling traffic <fetch_dir> <write_dir> <copy_bytes>
        HBM bytes per dispatch of every q4 kernel from one ``--pmc FETCH_SIZE``
        and one ``--pmc WRITE_SIZE`` run of ``bench.py --profile-pass``, each
        scaled by what the counter reads for the pass's calibration copy (an
        elementwise kernel that reads and writes ``copy_bytes`` bytes).

Both print short text meant for ``profiles/``.
"""
from __future__ import annotations

import csv
import glob
import os
import statistics
import sys
from collections import defaultdict

Q4_KERNELS = ("q4_gemv1_kernel", "q4_gemv1_step_kernel", "gemm_q4_kernel", "tile_kernel", "rmsnorm_kernel", "qkv_post_kernel",
              "attn_partial_kernel", "attn_merge_kernel", "add_norm_kernel", "embed_kernel", "head_kernel",
              "head_fold_kernel", "quant_kernel", "split_x_kernel", "split_fix_kernel", "q4_ffn1_kernel",
              "ffn1_sum_kernel", "ffn1_vdown_kernel")
CALIBRATION = "MulFunctor"  # the profile pass's copy: torch.mul(src, 1.0, out=dst)


def _short(name: str) -> str:
    name = name.replace("void ", "").replace("(anonymous namespace)::", "").replace("alv::", "")
    if "(" in name:
        name = name[: name.index("(")]
    return name


def _find(d: str, suffix: str) -> str:
    files = sorted(glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True))
    if not files:
        raise FileNotFoundError(f"no *{suffix} under {d}")
    return files[0]


def stats(d: str) -> str:
    """Kernel statistics of a --kernel-trace --stats run (all kernels, by time)."""
    rows = list(csv.DictReader(open(_find(d, "kernel_stats.csv"))))
    out = ["kernel | calls | avg us | min us | max us | total %"]
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        out.append(f"{_short(r['Name'])} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.3f} | "
                   f"{float(r['MinNs']) / 1e3:.3f} | {float(r['MaxNs']) / 1e3:.3f} | {float(r['Percentage']):.2f}")
    return "\n".join(out)


def launches(d: str) -> str:
    """Q4 kernel dispatches of a --kernel-trace run grouped by launch shape
    (kernel, grid, LDS bytes): one kernel instance serves several matrix
    shapes, and each shape has its own duration."""
    per = defaultdict(list)
    for r in csv.DictReader(open(_find(d, "kernel_trace.csv"))):
        name = _short(r["Kernel_Name"])
        if not any(q in name for q in Q4_KERNELS):
            continue
        grid = "x".join(str(int(r[f"Grid_Size_{a}"]) // max(1, int(r[f"Workgroup_Size_{a}"]))) for a in "XYZ")
        key = (name, grid, int(r["Workgroup_Size_X"]), int(r["LDS_Block_Size"]))
        per[key].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    out = ["kernel | workgroups (x*y*z) | threads | LDS B | calls | avg us | median us | min us"]
    for key, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        out.append(f"{key[0]} | {key[1]} | {key[2]} | {key[3]} | {len(v)} | {statistics.mean(v):.3f} | "
                   f"{statistics.median(v):.3f} | {min(v):.3f}")
    return "\n".join(out)


def _counter_means(d: str, counter: str) -> dict:
    """Mean of `counter` per dispatch, per kernel name."""
    per = defaultdict(lambda: defaultdict(float))
    for r in csv.DictReader(open(_find(d, "counter_collection.csv"))):
        if r["Counter_Name"] != counter:
            continue
        # one row per (dispatch, counter): sum the dimension instances of a dispatch
        per[_short(r["Kernel_Name"])][r.get("Dispatch_Id", r.get("Correlation_Id", ""))] += float(r["Counter_Value"])
    return {k: statistics.mean(v.values()) for k, v in per.items()}


def traffic(fetch_dir: str, write_dir: str, copy_bytes: int) -> str:
    fetch = _counter_means(fetch_dir, "FETCH_SIZE")
    write = _counter_means(write_dir, "WRITE_SIZE")
    cal = [k for k in fetch if CALIBRATION in k]
    if not cal:
        raise RuntimeError("calibration copy kernel not found in the FETCH_SIZE run")
    f_cal = fetch[cal[0]] * 1024.0
    w_cal = write[[k for k in write if CALIBRATION in k][0]] * 1024.0
    f_scale, w_scale = copy_bytes / f_cal, copy_bytes / w_cal
    out = [f"calibration: {cal[0]} reads and writes {copy_bytes} B; FETCH_SIZE reads {f_cal:.0f} B "
           f"(scale {f_scale:.4f}), WRITE_SIZE reads {w_cal:.0f} B (scale {w_scale:.4f})",
           "kernel | FETCH_SIZE KiB/dispatch | WRITE_SIZE KiB/dispatch | traffic B/dispatch (scaled)"]
    for k in sorted(fetch):
        if not any(q in k for q in Q4_KERNELS):
            continue
        t = fetch[k] * 1024.0 * f_scale + write.get(k, 0.0) * 1024.0 * w_scale
        out.append(f"{k} | {fetch[k]:.1f} | {write.get(k, 0.0):.1f} | {t:.0f}")
        out.append(f"traffic_bytes_per_launch[{k}]: {t:.0f}")
    return "\n".join(out)


def decode(d: str) -> str:
    """Median duration of each op of the decode step, the launches named by
    their order: the streaming GEMV with a fused residual step is the QKV or
    the gate/up launch (its instance: GLU or not), layer 0's QKV with the
    input norm when it follows the embedding, the LM head with the final
    residual step and norm when head_kernel follows it; without one, with
    256 workgroups it is the LM head after the final residual step (or layer
    0's QKV after the input norm), with 240 workgroups O after the attention
    merge or FFN down after the gate/up launch."""
    with open(_find(d, "kernel_trace.csv")) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    seq = []  # (tag, us) in launch order
    prev = None
    for r in rows:
        n = r["Kernel_Name"]
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
        wg = int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"]))
        if "attn_partial" in n:
            tag = "attention, global" if "512" in n else "attention, sliding"
        elif "attn_merge" in n:
            tag = "attention merge"
        elif "head_fold" in n:
            tag = "head fold"
        elif "head_kernel" in n:
            tag = "head softcap/argmax"
        elif "embed_kernel" in n:
            tag = "embedding"
        elif "add_norm_kernel" in n:
            tag = "final residual step + norm"
        elif "rmsnorm_kernel" in n:
            tag = "layer-0 input norm"
        elif "q4_ffn1_kernel" in n:
            tag = "FFN one launch + residual step" if "true, true>" in n else "FFN one launch"
        elif "ffn1_sum_kernel" in n:
            tag = "FFN partial sum"
        elif "q4_gemv1_step_kernel" in n:
            if "true, true, 1," in n:
                tag = "gate/up + residual step"
            else:
                tag = "QKV, layer 0 + input norm" if prev == "embedding" else "QKV + residual step"
        elif "q4_gemv1_kernel" in n and wg == 240:
            tag = "FFN down" if prev == "gate/up + residual step" else "O"
        elif "q4_gemv1_kernel" in n:
            tag = "LM-head GEMV" if prev == "final residual step + norm" else "QKV, layer 0"
        else:
            continue
        if tag == "head softcap/argmax" and seq and seq[-1][0] == "QKV + residual step":
            seq[-1] = ("LM-head GEMV + final residual step + norm", seq[-1][1])
        seq.append((tag, us))
        prev = tag
    out = defaultdict(list)
    for tag, us in seq:
        out[tag].append(us)
    lines = ["op | launches | median us | mean us"]
    for tag, v in out.items():
        lines.append(f"{tag} | {len(v)} | {statistics.median(v):.2f} | {statistics.mean(v):.2f}")
    return "\n".join(lines)


def counters(d: str) -> str:
    """Mean per dispatch of every counter of a --pmc run, per Q4 kernel, plus
    the ratios that matter here (LDS conflicts per access, MFMA and VALU busy
    fractions of the wave cycles' CU share)."""
    names = sorted({r["Counter_Name"] for r in csv.DictReader(open(_find(d, "counter_collection.csv")))})
    means = {c: _counter_means(d, c) for c in names}
    kernels = sorted({k for m in means.values() for k in m if any(q in k for q in Q4_KERNELS)})
    out = ["kernel | " + " | ".join(names)]
    for k in kernels:
        out.append(f"{k} | " + " | ".join(f"{means[c].get(k, float('nan')):.4g}" for c in names))
    return "\n".join(out)


def read_traffic(path: str, kernel: str):
    """The scaled traffic of `kernel` from a committed traffic summary, or None."""
    if not os.path.exists(path):
        return None
    key = f"traffic_bytes_per_launch[{kernel}]:"
    for line in open(path):
        if line.startswith(key):
            return int(float(line[len(key):]))
    return None


def main(argv) -> int:
    if len(argv) >= 2 and argv[0] == "stats":
        print(stats(argv[1]))
        return 0
    if len(argv) >= 2 and argv[0] == "launches":
        print(launches(argv[1]))
        return 0
    if len(argv) >= 2 and argv[0] == "decode":
        print(decode(argv[1]))
        return 0
    if len(argv) >= 2 and argv[0] == "counters":
        print(counters(argv[1]))
        return 0
    if len(argv) >= 4 and argv[0] == "traffic":
        print(traffic(argv[1], argv[2], int(argv[3])))
        return 0
    print(__doc__, file=sys.stderr)
    return 2


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
