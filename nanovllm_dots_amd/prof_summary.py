"""Summaries of rocprofv3 CSV output for the FM head's kernels.

    python -m nanovllm_dots_amd.prof_summary stats <run_kernel_stats.csv>
    python -m nanovllm_dots_amd.prof_summary pmc <fetch counter csv> <write counter csv> --calib-mib 256
    python -m nanovllm_dots_amd.prof_summary mfma <counter csv> [--simds 1024]

``stats`` tabulates ``rocprofv3 --kernel-trace --stats`` per kernel, with the
role each GEMM instantiation plays in a DiT block. ``pmc`` reads one
``--pmc FETCH_SIZE`` run and one ``--pmc WRITE_SIZE`` run of the same program,
calibrates both counters against the device copy of known size that
``bench.py --calib-copy-mib`` issues first (the largest ``copyBuffer``
dispatch: it reads and writes ``calib-mib`` MiB), and reports HBM bytes per
dispatch per role. Roles follow dispatch order within a block: the gate-residual
GEMM that follows attention is the O projection, the one that follows the
GELU GEMM is fc2.
"""
from __future__ import annotations

import argparse
import collections
import csv
import re
import statistics
import sys

_EPI = re.compile(r"OpBf16, (\d+)>")


def short_name(name: str) -> str:
    name = name.replace("dfh::(anonymous namespace)::", "")
    name = re.sub(r"\(.*\)$", "", name)
    return name.replace("void ", "")


def roles(names):
    """Role of each dispatch of a sequence of kernel names (dispatch order)."""
    out = []
    prev = ""
    for n in names:
        s = short_name(n)
        m = _EPI.search(s) if s.startswith("gemm_mfma_kernel") else None
        if m:
            epi = int(m.group(1))
            r = {3: "qkv_gemm", 1: "fc1_gemm"}.get(epi)
            if epi == 2:
                r = "fc2_gemm" if prev == "fc1_gemm" else "o_gemm"
            if r is None:
                r = "gemm_epi%d" % epi
        elif s.startswith("seq_attention"):
            r = "attention"
        elif s.startswith("decode_attention") or s.startswith("decode_combine"):
            r = "decode_attention"
        elif s.startswith("ln_modulate"):
            r = "ln_modulate"
        else:
            r = s
        out.append(r)
        prev = r
    return out


def stats(path: str, top: int = 16) -> str:
    rows = list(csv.DictReader(open(path)))
    total = sum(float(r["TotalDurationNs"]) for r in rows)
    lines = ["| kernel | calls | avg us | total ms | % |", "|---|---:|---:|---:|---:|"]
    for r in rows[:top]:
        lines.append("| `%s` | %s | %.1f | %.2f | %.2f |" % (
            short_name(r["Name"])[:100], r["Calls"], float(r["AverageNs"]) / 1e3,
            float(r["TotalDurationNs"]) / 1e6, 100 * float(r["TotalDurationNs"]) / total))
    return "\n".join(lines)


def _load(path: str):
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Dispatch_Id"]))
    return [(r["Kernel_Name"], float(r["Counter_Value"])) for r in rows]


def pmc(fetch_csv: str, write_csv: str, calib_mib: int):
    calib = calib_mib * 1024.0  # KiB read and written by the calibration copy
    out = {}
    factors = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        rows = _load(path)
        copies = [v for n, v in rows if "copyBuffer" in n]
        if not copies:
            raise SystemExit(f"{path}: no calibration copy dispatch")
        factors[counter] = calib / max(copies)
        by_role = collections.defaultdict(list)
        for role, (_, v) in zip(roles([n for n, _ in rows]), rows):
            by_role[role].append(v)
        out[counter] = by_role
    return factors, out


def pmc_table(factors, out, roles_wanted=("qkv_gemm", "o_gemm", "fc1_gemm", "fc2_gemm", "attention",
                                          "ln_modulate")) -> str:
    lines = ["| role | dispatches | FETCH_SIZE KiB (raw median) | WRITE_SIZE KiB (raw median) | "
             "HBM read MB | HBM write MB | HBM total MB |", "|---|---:|---:|---:|---:|---:|---:|"]
    machine = []
    for role in roles_wanted:
        f = out["FETCH_SIZE"].get(role)
        w = out["WRITE_SIZE"].get(role)
        if not f or not w:
            continue
        fk, wk = statistics.median(f), statistics.median(w)
        rb = fk * 1024 * factors["FETCH_SIZE"]
        wb = wk * 1024 * factors["WRITE_SIZE"]
        lines.append("| %s | %d | %.1f | %.1f | %.1f | %.1f | %.1f |" % (
            role, len(f), fk, wk, rb / 1e6, wb / 1e6, (rb + wb) / 1e6))
        machine.append("traffic_bytes_per_launch %s %d" % (role, round(rb + wb)))
    return "\n".join(lines), machine


# SQ counters are summed over shader engines and XCDs; GRBM_GUI_ACTIVE is summed over the XCDs
MFMA_COUNTERS = ("GRBM_GUI_ACTIVE", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_INSTS_MFMA",
                 "SQ_INSTS_VALU", "SQ_ACTIVE_INST_VALU", "SQ_BUSY_CU_CYCLES", "SQ_INSTS_VALU_TRANS_F32")


def mfma(path: str, simds: int = 1024, xcds: int = 8):
    """Per-role medians of one multi-counter ``--pmc`` run.

    mfma_util = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE per XCD * SIMDs), the
    expression of rocprofv3's derived ``MfmaUtil``; clock = GRBM_GUI_ACTIVE per XCD /
    dispatch duration; bf16 MFMA FLOP = SQ_INSTS_VALU_MFMA_MOPS_BF16 * 512.
    """
    per = collections.defaultdict(dict)
    meta = {}
    for r in csv.DictReader(open(path)):
        d = int(r["Dispatch_Id"])
        per[d][r["Counter_Name"]] = per[d].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        dur = None
        if r.get("Start_Timestamp") and r.get("End_Timestamp"):
            dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9
        meta[d] = (r["Kernel_Name"], dur, r.get("Arch_VGPR_Count") or r.get("VGPR_Count"),
                   r.get("Accum_VGPR_Count"))
    ids = sorted(per)
    rl = roles([meta[d][0] for d in ids])
    by = collections.defaultdict(list)
    for role, d in zip(rl, ids):
        c = per[d]
        gui = c.get("GRBM_GUI_ACTIVE", 0.0) / xcds
        if gui <= 0:
            continue
        name, dur, vg, ag = meta[d]
        row = {
            "cycles": gui,
            "mfma_util": c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (gui * simds),
            "mfma_flop": c.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0) * 512,
            "mfma_iop": c.get("SQ_INSTS_VALU_MFMA_MOPS_I8", 0.0) * 512,
            "mfma_insts": c.get("SQ_INSTS_MFMA", 0.0),
            "valu_insts": c.get("SQ_INSTS_VALU", 0.0),
            "trans_insts": c.get("SQ_INSTS_VALU_TRANS_F32", 0.0),
            # quad-cycles summed over the SIMDs -> fraction of SIMD cycles with a VALU op in flight
            "valu_busy": c.get("SQ_ACTIVE_INST_VALU", 0.0) * 4 / (gui * simds),
            "cu_busy": c.get("SQ_BUSY_CU_CYCLES", 0.0) * 4 / (gui * simds / 4),
            "clock_ghz": gui / dur / 1e9 if dur else float("nan"),
            "vgpr": vg, "agpr": ag,
        }
        by[role].append(row)
    return by


def mfma_table(by, roles_wanted=("qkv_gemm", "o_gemm", "fc1_gemm", "fc2_gemm", "attention", "ln_modulate")) -> str:
    """Per-role medians; roles_wanted=None lists every role (kernel) that ran."""
    if roles_wanted is None:
        roles_wanted = sorted(by)
    if any(r["mfma_iop"] for rows in by.values() for r in rows):
        return _mfma_table_i8(by, roles_wanted)
    lines = ["| role | dispatches | cycles (per XCD) | clock GHz | MFMA busy | bf16 MFMA GFLOP | MFMA insts (M) | "
             "VALU insts (M) | of which transc. (M) | VALU busy | VGPR / AGPR |",
             "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---|"]
    for role in roles_wanted:
        rows = by.get(role)
        if not rows:
            continue
        med = lambda k: statistics.median(r[k] for r in rows)
        lines.append("| %s | %d | %.0f | %.2f | %.1f %% | %.1f | %.2f | %.2f | %.2f | %.1f %% | %s / %s |" % (
            role, len(rows), med("cycles"), med("clock_ghz"), 100 * med("mfma_util"), med("mfma_flop") / 1e9,
            med("mfma_insts") / 1e6, med("valu_insts") / 1e6, med("trans_insts") / 1e6, 100 * med("valu_busy"),
            rows[0]["vgpr"], rows[0]["agpr"]))
    return "\n".join(lines)


def _mfma_table_i8(by, roles_wanted) -> str:
    lines = ["| kernel | dispatches | cycles (per XCD) | MFMA busy | int8 MFMA GOP | bf16 MFMA GFLOP | VALU busy |",
             "|---|---:|---:|---:|---:|---:|---:|"]
    for role in roles_wanted:
        rows = by.get(role)
        if not rows:
            continue
        med = lambda k: statistics.median(r[k] for r in rows)
        lines.append("| `%s` | %d | %.0f | %.1f %% | %.1f | %.1f | %.1f %% |" % (
            role[:90], len(rows), med("cycles"), 100 * med("mfma_util"), med("mfma_iop") / 1e9,
            med("mfma_flop") / 1e9, 100 * med("valu_busy")))
    return "\n".join(lines)


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("--top", type=int, default=16)
    p = sub.add_parser("pmc")
    p.add_argument("fetch_csv")
    p.add_argument("write_csv")
    p.add_argument("--calib-mib", type=int, required=True)
    q = sub.add_parser("mfma")
    q.add_argument("csv")
    q.add_argument("--simds", type=int, default=1024)
    q.add_argument("--all", action="store_true", help="every kernel, not only the DiT roles")
    a = ap.parse_args(argv)
    if a.cmd == "stats":
        print(stats(a.csv, a.top))
    elif a.cmd == "mfma":
        print(mfma_table(mfma(a.csv, a.simds), None if a.all else mfma_table.__defaults__[0]))
    else:
        factors, out = pmc(a.fetch_csv, a.write_csv, a.calib_mib)
        table, machine = pmc_table(factors, out)
        print("calibration: FETCH_SIZE x %.4f, WRITE_SIZE x %.4f (bytes per counted KiB / 1024)" % (
            factors["FETCH_SIZE"], factors["WRITE_SIZE"]))
        print()
        print(table)
        print()
        print("```")
        print("\n".join(machine))
        print("```")


if __name__ == "__main__":
    sys.exit(main())
