#!/usr/bin/env python3
"""Throughput of the ntops hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--ops all|name,...]

A step is one pass of an op over its full synthetic workload (the shapes
below), inputs resident in HBM.  The headline line is rms_norm on bf16
(16384, 4096) -- the configuration the metric is quoted on -- and the same
JSON line carries every other workload under "ops".

Timing: W eager warmup steps, then K steps captured in one HIP graph (so host
launch overhead does not pad ~35 us kernels), replayed R times (--replays,
default 5) back to back between HIP events recorded on the launch stream;
the reported time per step is the median over the R replays (each replay's
figure and the spread are in the line too).  Before the timed replays the
graph is replayed untimed for --settle-ms of wall time (default 100): the
part's clocks take ~10 ms to settle after a change of load (bmm bf16
32 x (2048 x 128)(128 x 2048) ran 63-88 us per step in the first replays
after an MFMA-heavy workload or an idle second, 53-58 us once settled), so
without it the short workloads were timed inside that transient.  Three input/output buffer sets
rotate so the 256 MB MALL cannot serve a step from the previous one.
Achieved bandwidth uses algorithmic bytes (every compulsory byte counted
once); GEMMs report algorithmic flops.  A plain streaming copy (ntops_cast
f32 -> f32) runs as its own workload and gives each bandwidth-bound op its
fraction of the measured ceiling; torch.mm / torch.bmm (hipBLASLt, eager),
torch's GPU scaled_dot_product_attention (flash / memory-efficient backends)
and conv2d (MIOpen) are timed at their configs as same-box yardsticks, and
Tensor.copy_ beside the copy.  cpu_baseline times
PyTorch's CPU implementation of the same op (the reference the configs name)
on a bounded sample of the workload on this host's cores.
"""

import argparse
import json
import math
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "achieved HBM GB/s (% peak) for norm/softmax/RoPE/eltwise; bf16 mm TFLOP/s"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
NSETS = 3


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--replays", type=int, default=5, help="timed replays of the K-step graph (median reported)")
    p.add_argument("--settle-ms", type=float, default=100.0,
                   help="untimed replays of the captured steps for this much wall time before timing")
    p.add_argument("--ops", default="all")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    p.add_argument("--eager", action="store_true", help="time eager wrapper calls instead of a graph")
    p.add_argument("--copy-calibration", action="store_true",
                   help="run 10 plain 128 MiB copies (ntops_cast f32->f32) for byte-counter calibration")
    p.add_argument("--rocprof-summary", metavar="DB", help="print kernel-duration stats of a rocprofv3 database")
    p.add_argument("--traffic", metavar="DIR",
                   help="print calibrated HBM bytes per launch (JSON) from rocprofv3 --pmc databases in "
                        "DIR/<workload>_{FETCH,WRITE}_SIZE/ and DIR/cal_{FETCH,WRITE}_SIZE/")
    p.add_argument("--traffic-file", default=os.path.join(ROOT, "profiles", "traffic.json"),
                   help="measured HBM bytes per launch used to fill roofline.traffic")
    p.add_argument("--mfma", metavar="DIR",
                   help="print MFMA utilisation per GEMM workload (JSON) from rocprofv3 --pmc databases in "
                        "DIR/<workload>_<counter>/")
    p.add_argument("--counters", metavar="DB",
                   help="print, per kernel of a rocprofv3 --pmc database, the median of each counter and its "
                        "rate per CU per active cycle (markdown); --kernels limits the kernels by name fragment")
    p.add_argument("--kernels", default="", help="comma-separated kernel name fragments for --counters")
    p.add_argument("--mfma-file", default=os.path.join(ROOT, "profiles", "mfma.json"),
                   help="measured MFMA utilisation used to fill roofline.mfma_busy")
    return p.parse_args()


# ------------------------------------------------- rocprofv3 post-processing


def _db_rows(db, sql):
    import sqlite3

    con = sqlite3.connect(db)
    try:
        return con.execute(sql).fetchall()
    finally:
        con.close()


def _kernel_key(name):
    """Short stable key of a kernel symbol (template arguments kept)."""
    import re

    n = re.sub(r"\(anonymous namespace\)::", "", name)
    n = n.replace("ntops::", "")
    return n[:160]


def rocprof_summary(db):
    rows = _db_rows(db, "select name, duration from kernels")
    by = {}
    for n, d in rows:
        by.setdefault(_kernel_key(n), []).append(d / 1e3)
    print("| kernel | calls | mean us | median us | min us | max us |")
    print("|---|---|---|---|---|---|")
    for n, ds in sorted(by.items(), key=lambda kv: -sum(kv[1])):
        print(f"| `{n}` | {len(ds)} | {statistics.mean(ds):.2f} | {statistics.median(ds):.2f} | "
              f"{min(ds):.2f} | {max(ds):.2f} |")


def _counter_means(db):
    rows = _db_rows(db, "select kernel_name, counter_name, value, dispatch_id from counters_collection")
    per = {}
    for n, c, v, d in rows:
        per.setdefault((_kernel_key(n), c), {}).setdefault(d, 0.0)
        per[(_kernel_key(n), c)][d] += v
    return {k: statistics.mean(v.values()) for k, v in per.items()}


COPY_CAL_BYTES = 128 << 20


def _one_db(d):
    import glob

    dbs = sorted(glob.glob(os.path.join(d, "*.db")))
    assert dbs, f"no rocprofv3 database in {d}"
    return dbs[0]


def _counter_for(db, counter, pattern):
    vals = [v for (k, c), v in _counter_means(db).items() if c == counter and pattern in k]
    return statistics.mean(vals) if vals else None


def traffic(directory):
    """HBM bytes per launch of each workload's kernel: FETCH_SIZE and
    WRITE_SIZE (KiB per dispatch) each scaled by true_bytes / counter_bytes of
    a plain 128 MiB copy kernel (the calibration run)."""
    cal_f = _counter_for(_one_db(os.path.join(directory, "cal_FETCH_SIZE")), "FETCH_SIZE", "k_cast_pack")
    cal_w = _counter_for(_one_db(os.path.join(directory, "cal_WRITE_SIZE")), "WRITE_SIZE", "k_cast_pack")
    fetch_factor = COPY_CAL_BYTES / (cal_f * 1024)
    write_factor = COPY_CAL_BYTES / (cal_w * 1024)
    out = {"fetch_factor": round(fetch_factor, 4), "write_factor": round(write_factor, 4), "kernels": {}}
    for name, pattern in KERNEL_OF.items():
        fd, wd = os.path.join(directory, f"{name}_FETCH_SIZE"), os.path.join(directory, f"{name}_WRITE_SIZE")
        if not (os.path.isdir(fd) and os.path.isdir(wd)):
            continue
        f = _counter_for(_one_db(fd), "FETCH_SIZE", pattern)
        w = _counter_for(_one_db(wd), "WRITE_SIZE", pattern)
        if f is None or w is None:
            continue
        rd, wr = f * 1024 * fetch_factor, w * 1024 * write_factor
        out["kernels"][name] = {"kernel": pattern, "read_bytes": round(rd), "write_bytes": round(wr),
                                "bytes": round(rd + wr)}
    print(json.dumps(out, indent=1))


def _gpu_agent(db):
    """(num_xcc, cu_count) of the GPU agent recorded in a rocprofv3 database."""
    for (ext,) in _db_rows(db, "select extdata from rocpd_info_agent where type = 'GPU'"):
        info = json.loads(ext)
        return int(info.get("num_xcc", 8)), int(info.get("cu_count", 256))
    return 8, 256


def counter_table(db, fragments):
    """Markdown table of a --pmc database: per kernel (matched by name
    fragment), the median over dispatches of each counter, its value per CU
    per active cycle (GRBM_GUI_ACTIVE per XCD), the kernel time and the clock
    those imply."""
    nxcc, cus = _gpu_agent(db)
    frags = [f for f in fragments.split(",") if f] or [""]
    per = {}
    for kname, cname, v, disp, dur in _db_rows(
            db, "select kernel_name, counter_name, value, dispatch_id, duration from counters_collection"):
        key = _kernel_key(kname)
        f = next((f for f in frags if f in key), None)
        if f is None:
            continue
        per.setdefault((key, f), {}).setdefault(disp, {"duration": dur})[cname] = v
    for (key, f), disps in sorted(per.items(), key=lambda kv: kv[0][1]):
        rows = list(disps.values())
        counters = sorted({c for r in rows for c in r if c != "duration"})
        med = {c: statistics.median(r[c] for r in rows if c in r) for c in counters}
        dur = statistics.median(r["duration"] for r in rows)
        gui = med.get("GRBM_GUI_ACTIVE")
        head = f"`{key[:90]}`: {len(rows)} dispatches, {dur / 1e3:.1f} us"
        if gui:
            head += f", {gui / nxcc:.0f} active cycles per XCD, {gui / nxcc / dur:.2f} GHz"
        print(f"{head}\n\n| counter | median per dispatch | per CU per active cycle |\n|---|---|---|")
        for c in counters:
            if c == "GRBM_GUI_ACTIVE":
                continue
            rate = f"{med[c] / (gui / nxcc * cus):.3f}" if gui else ""
            print(f"| {c} | {med[c]:.0f} | {rate} |")
        print()


def mfma_report(directory):
    """Matrix-core utilisation of each matrix workload's kernel from one
    rocprofv3 pass of SQ_INSTS_VALU_MFMA_MOPS_BF16, SQ_VALU_MFMA_BUSY_CYCLES
    and GRBM_GUI_ACTIVE in DIR/<workload>_mfma/.  flops = MOPS * 512 (checked
    against the algorithmic count); busy = MFMA busy cycles / (active cycles
    per XCD * 4 SIMDs * CUs); clock = active cycles per XCD / kernel time."""
    out = {"kernels": {}}
    for name in ("mm", "addmm", "bmm", "sdpa", "conv2d", "mfma_ceiling"):
        d = os.path.join(directory, f"{name}_mfma")
        if not os.path.isdir(d):
            continue
        db = _one_db(d)
        nxcc, cus = _gpu_agent(db)
        pattern = KERNEL_OF[name]
        per = {}
        for kname, cname, v, disp, dur in _db_rows(
                db, "select kernel_name, counter_name, value, dispatch_id, duration from counters_collection"):
            if pattern in _kernel_key(kname):
                per.setdefault(disp, {"duration": dur})[cname] = v
        rows = [r for r in per.values() if {"SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_VALU_MFMA_BUSY_CYCLES",
                                            "GRBM_GUI_ACTIVE"} <= set(r)]
        if not rows:
            continue
        busy = [r["SQ_VALU_MFMA_BUSY_CYCLES"] / (r["GRBM_GUI_ACTIVE"] / nxcc * 4 * cus) for r in rows]
        clock = [r["GRBM_GUI_ACTIVE"] / nxcc / r["duration"] for r in rows]
        out["kernels"][name] = {
            "kernel": pattern,
            "dispatches": len(rows),
            "flops": round(statistics.median(r["SQ_INSTS_VALU_MFMA_MOPS_BF16"] for r in rows) * 512),
            "busy": round(statistics.median(busy), 4),
            "clock_ghz": round(statistics.median(clock), 3),
            "kernel_us": round(statistics.median(r["duration"] for r in rows) / 1e3, 2),
        }
    print(json.dumps(out, indent=1))


# kernel symbol fragment of each workload's dominant kernel
KERNEL_OF = {
    "copy": "k_cast_pack",
    "mfma_ceiling": "k_mfma_probe",
    "silu": "k_unary_dense",
    "add": "k_binary_dense",
    "gelu_f32": "k_unary_dense",
    "gelu_bf16": "k_unary_dense",
    "exp_f32": "k_unary_dense",
    "exp_bf16": "k_unary_dense",
    "bitwise_and": "k_binary_dense",
    "im2col": "k_im2col",
    "div": "k_binary_dense",
    "eq": "k_binary_dense",
    "clamp": "k_clamp_dense",
    "copy_half": "k_cast_pack",
    "rms_norm": "k_rms_vec",
    "layer_norm": "k_ln_vec",
    "rms_norm_odd": "k_rms_odd",
    "rms_norm_wide": "k_rms_wide",
    "softmax_wide": "k_softmax_wide",
    "softmax": "k_softmax_vec",
    "rope": "k_rope_half_vec",
    "rope_qk": "k_rope_half_vec",
    "add_rms_norm": "k_add_rms_vec",
    "mm": "k_gemm_mfma",
    "addmm": "k_gemm_mfma",
    "bmm": "k_gemm_panel",
    "sdpa": "k_flash_attn",
    "conv2d": "k_gemm_mfma",
}


def copy_calibration():
    import ctypes

    from ntops_amd import _lib

    lib = _lib.load()
    n = COPY_CAL_BYTES // 4
    xs = [torch.randn(n, device="cuda") for _ in range(NSETS)]
    ys = [torch.empty(n, device="cuda") for _ in range(NSETS)]
    shape, st = _lib.i64_array((n,)), _lib.i64_array((1,))
    torch.cuda.synchronize()
    for i in range(10):
        _lib.check(lib.ntops_cast(_lib.F32, _lib.F32, 1, shape, xs[i % NSETS].data_ptr(), st,
                                  ys[i % NSETS].data_ptr(), st,
                                  ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "copy")
    torch.cuda.synchronize()
    print(f"copy calibration: 10 x {COPY_CAL_BYTES} B (ntops_cast f32 -> f32, k_cast_pack<float, float>)")


def load_traffic(path):
    try:
        with open(path) as f:
            return json.load(f).get("kernels", {})
    except (OSError, ValueError):
        return {}


# ----------------------------------------------------------- workloads ----


class Workload:
    """name, description, algorithmic work per step, and callables that build
    rotating GPU buffer sets, launch one step on a set, and time the torch
    CPU reference on a sample."""

    def __init__(self, name, desc, unit, bound, work, kernels_per_step, build, step, cpu, dtype):
        self.name, self.desc, self.unit, self.bound = name, desc, unit, bound
        self.work, self.kernels_per_step = work, kernels_per_step
        self.build, self.step, self.cpu, self.dtype = build, step, cpu, dtype


def _gen(seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return g


def _cpu_gen(seed=0):
    return torch.Generator().manual_seed(seed)


def make_workloads():
    import torch.nn.functional as F

    import ntops_amd
    from ntops_amd import _lib
    from ntops_amd.torch._gemm import gemm
    from ntops_amd.torch.utils import _unary

    lib = _lib.load()

    import ctypes

    def stream():
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def check(rc, what):
        _lib.check(rc, what)

    W = []

    # silu fp32 (8192, 4096)
    def silu_build(i):
        x = torch.randn(8192, 4096, device="cuda", generator=_gen(i))
        return {"x": x, "y": torch.empty_like(x)}

    def silu_step(s):
        _unary(_lib.UNARY_SILU, s["x"], s["y"], "silu")

    def silu_cpu():
        x = torch.randn(2048, 4096, generator=_cpu_gen())
        return (lambda: F.silu(x)), 2 * x.numel() * 4, "F.silu fp32 (2048, 4096) = 1/4 of the workload"

    W.append(Workload("silu", "silu fp32 (8192, 4096)", "GB/s", "hbm", 2 * 8192 * 4096 * 4, 1,
                      silu_build, silu_step, silu_cpu, "f32"))

    # the rest of the elementwise family: one workload per kernel shape --
    # two tensors in (div floor), bool out (eq), four operands (clamp)
    EN = (8192, 4096)
    en_shape, en_strides = _lib.i64_array(EN), _lib.i64_array((EN[1], 1))

    def ew_build(i, n_in):
        g = _gen(50 + i)
        ts = [torch.randn(*EN, device="cuda", generator=g) for _ in range(n_in)]
        return {"in": ts, "y": torch.empty(*EN, device="cuda"), "yb": torch.empty(*EN, dtype=torch.bool, device="cuda")}

    def div_step(s):
        a, b = s["in"]
        check(lib.ntops_binary(_lib.BINARY_DIV_FLOOR, _lib.F32, 2, en_shape, a.data_ptr(), en_strides, b.data_ptr(),
                               en_strides, 0.0, 0, 1.0, 1, s["y"].data_ptr(), en_strides, stream()), "div")

    def eq_step(s):
        a, b = s["in"]
        check(lib.ntops_compare(_lib.CMP_EQ, _lib.F32, 2, en_shape, a.data_ptr(), en_strides, b.data_ptr(),
                                en_strides, 0.0, 0, s["yb"].data_ptr(), en_strides, stream()), "eq")

    def clamp_step(s):
        x, lo, hi = s["in"]
        check(lib.ntops_clamp(_lib.F32, 2, en_shape, x.data_ptr(), en_strides, lo.data_ptr(), en_strides, 0.0, 0, 1,
                              hi.data_ptr(), en_strides, 0.0, 0, 1, s["y"].data_ptr(), en_strides, stream()), "clamp")

    def ew_cpu(fn, n_in, bytes_per_el, desc):
        def make():
            g = _cpu_gen()
            ts = [torch.randn(2048, 4096, generator=g) for _ in range(n_in)]
            return (lambda: fn(*ts)), 2048 * 4096 * bytes_per_el, desc
        return make

    W.append(Workload("div", "div fp32 (8192, 4096) / (8192, 4096), rounding_mode='floor'", "GB/s", "hbm",
                      12 * EN[0] * EN[1], 1, lambda i: ew_build(i, 2), div_step,
                      ew_cpu(lambda a, b: torch.div(a, b, rounding_mode="floor"), 2, 12,
                             "torch.div(rounding_mode='floor') fp32 (2048, 4096) = 1/4 of the workload"), "f32"))
    W.append(Workload("eq", "eq fp32 (8192, 4096) == (8192, 4096) -> bool", "GB/s", "hbm",
                      9 * EN[0] * EN[1], 1, lambda i: ew_build(i, 2), eq_step,
                      ew_cpu(torch.eq, 2, 9, "torch.eq fp32 (2048, 4096) = 1/4 of the workload"), "f32"))
    W.append(Workload("clamp", "clamp fp32 (8192, 4096) with tensor min and max", "GB/s", "hbm",
                      16 * EN[0] * EN[1], 1, lambda i: ew_build(i, 3), clamp_step,
                      ew_cpu(torch.clamp, 3, 16, "torch.clamp fp32 (2048, 4096), tensor bounds = 1/4 of the workload"),
                      "f32"))

    # the rest of the hot-path elementwise rows at (8192, 4096): add (three
    # bf16 streams), gelu and exp in fp32 and bf16, bitwise_and on int32
    def ew_dt_build(i, n_in, dtype):
        g = _gen(60 + i)
        if dtype == torch.int32:
            ts = [torch.randint(-2**31, 2**31 - 1, EN, device="cuda", generator=g, dtype=torch.int32)
                  for _ in range(n_in)]
        else:
            ts = [torch.randn(*EN, device="cuda", generator=g).to(dtype) for _ in range(n_in)]
        return {"in": ts, "y": torch.empty(*EN, device="cuda", dtype=dtype)}

    def unary_step(op, code):
        def step(s):
            check(lib.ntops_unary(op, code, 2, en_shape, s["in"][0].data_ptr(), en_strides, s["y"].data_ptr(),
                                  en_strides, stream()), "unary")
        return step

    def binary_step(op, code):
        def step(s):
            a, b = s["in"]
            check(lib.ntops_binary(op, code, 2, en_shape, a.data_ptr(), en_strides, b.data_ptr(), en_strides,
                                   0.0, 0, 1.0, 1, s["y"].data_ptr(), en_strides, stream()), "binary")
        return step

    def ew_dt_cpu(fn, n_in, dtype, bytes_per_el, desc):
        def make():
            g = _cpu_gen()
            if dtype == torch.int32:
                ts = [torch.randint(-2**31, 2**31 - 1, (2048, 4096), generator=g, dtype=torch.int32)
                      for _ in range(n_in)]
            else:
                ts = [torch.randn(2048, 4096, generator=g).to(dtype) for _ in range(n_in)]
            return (lambda: fn(*ts)), 2048 * 4096 * bytes_per_el, desc + " (2048, 4096) = 1/4 of the workload"
        return make

    n_el = EN[0] * EN[1]
    W.append(Workload("add", "add bf16 (8192, 4096) + (8192, 4096), alpha 1", "GB/s", "hbm", 6 * n_el, 1,
                      lambda i: ew_dt_build(i, 2, torch.bfloat16), binary_step(_lib.BINARY_ADD, _lib.BF16),
                      ew_dt_cpu(torch.add, 2, torch.bfloat16, 6, "torch.add bf16"), "bf16"))
    for nm, op, fn in (("gelu", _lib.UNARY_GELU, F.gelu), ("exp", _lib.UNARY_EXP, torch.exp)):
        for dtype, code, tag, esz in ((torch.float32, _lib.F32, "f32", 4), (torch.bfloat16, _lib.BF16, "bf16", 2)):
            W.append(Workload(f"{nm}_{tag}", f"{nm} {'fp32' if tag == 'f32' else 'bf16'} (8192, 4096)", "GB/s", "hbm",
                              2 * esz * n_el, 1, (lambda dt: lambda i: ew_dt_build(i, 1, dt))(dtype),
                              unary_step(op, code), ew_dt_cpu(fn, 1, dtype, 2 * esz, f"{fn.__name__} {tag}"), tag))
    W.append(Workload("bitwise_and", "bitwise_and int32 (8192, 4096) & (8192, 4096)", "GB/s", "hbm", 12 * n_el, 1,
                      lambda i: ew_dt_build(i, 2, torch.int32), binary_step(_lib.BINARY_BITWISE_AND, _lib.I32),
                      ew_dt_cpu(torch.bitwise_and, 2, torch.int32, 12, "torch.bitwise_and int32"), "int32"))

    # streaming copy (ntops_cast f32 -> f32, 128 MiB in and out per step):
    # the measured ceiling of the bandwidth-bound kernels
    CN_ = 32 << 20
    cp_shape, cp_st = _lib.i64_array((CN_,)), _lib.i64_array((1,))

    def copy_build(i):
        x = torch.randn(CN_, device="cuda", generator=_gen(80 + i))
        return {"x": x, "y": torch.empty_like(x)}

    def copy_step(s):
        check(lib.ntops_cast(_lib.F32, _lib.F32, 1, cp_shape, s["x"].data_ptr(), cp_st, s["y"].data_ptr(), cp_st,
                             stream()), "copy")

    def copy_cpu():
        x = torch.randn(CN_ // 4, generator=_cpu_gen())
        y = torch.empty_like(x)
        return (lambda: y.copy_(x)), 2 * x.numel() * 4, "Tensor.copy_ fp32 32 MiB = 1/4 of the workload"

    W.append(Workload("copy", "streaming copy fp32 128 MiB -> 128 MiB (ntops_cast): measured HBM ceiling", "GB/s",
                      "hbm", 2 * CN_ * 4, 1, copy_build, copy_step, copy_cpu, "f32"))
    W[-1].yardstick = (lambda s: s["y"].copy_(s["x"]), "torch Tensor.copy_ (device-to-device), eager")

    # the same copy at half the size (64 MiB each way): the ceiling of the
    # bf16 (8192, 4096) elementwise workloads, whose launches are this short
    cp2_shape = _lib.i64_array((CN_ // 2,))

    def copy_half_build(i):
        x = torch.randn(CN_ // 2, device="cuda", generator=_gen(90 + i))
        return {"x": x, "y": torch.empty_like(x)}

    def copy_half_step(s):
        check(lib.ntops_cast(_lib.F32, _lib.F32, 1, cp2_shape, s["x"].data_ptr(), cp_st, s["y"].data_ptr(), cp_st,
                             stream()), "copy")

    W.append(Workload("copy_half", "streaming copy fp32 64 MiB -> 64 MiB (ntops_cast): the ceiling at half size",
                      "GB/s", "hbm", CN_ * 4, 1, copy_half_build, copy_half_step, None, "f32"))

    # matrix-core rate probe: full-chip bf16 MFMAs on register operands, the
    # measured ceiling of the matrix-bound kernels
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    PROBE_ITERS = 5600

    def probe_build(i):
        return {"out": torch.empty(cus * 4, device="cuda")}

    def probe_step(s):
        check(lib.ntops_mfma_rate_probe(cus, PROBE_ITERS, s["out"].data_ptr(), stream()), "mfma probe")

    W.append(Workload("mfma_ceiling", f"bf16 MFMA rate probe: {cus} workgroups x 4 waves x {PROBE_ITERS} rounds of "
                      "8 v_mfma_f32_32x32x16_bf16 on register operands: measured matrix-core ceiling", "TFLOP/s",
                      "mfma", cus * 4 * PROBE_ITERS * 8 * 32768, 1, probe_build, probe_step, None, "bf16"))

    # rms_norm / layer_norm bf16 (16384, 4096)
    R, C = 16384, 4096

    def norm_build(i):
        g = _gen(100 + i)
        x = torch.randn(R, C, device="cuda", generator=g).bfloat16()
        w = (1 + 0.02 * torch.randn(C, device="cuda", generator=g)).bfloat16()
        b = (0.02 * torch.randn(C, device="cuda", generator=g)).bfloat16()
        return {"x": x, "w": w, "b": b, "y": torch.empty_like(x)}

    def rms_step(s):
        check(lib.ntops_rms_norm(_lib.BF16, R, C, s["x"].data_ptr(), C, s["w"].data_ptr(), 0, _lib.BF16, 1e-6,
                                 s["y"].data_ptr(), C, stream()), "rms_norm")

    def ln_step(s):
        check(lib.ntops_layer_norm(_lib.BF16, R, C, s["x"].data_ptr(), C, s["w"].data_ptr(), s["b"].data_ptr(), 0,
                                   _lib.BF16, 1e-5, s["y"].data_ptr(), C, stream()), "layer_norm")

    def norm_cpu_inputs():
        g = _cpu_gen()
        x = torch.randn(4096, C, generator=g).bfloat16()
        w = (1 + 0.02 * torch.randn(C, generator=g)).bfloat16()
        b = (0.02 * torch.randn(C, generator=g)).bfloat16()
        return x, w, b

    def rms_cpu():
        x, w, _ = norm_cpu_inputs()
        return (lambda: F.rms_norm(x, (C,), w, 1e-6)), 2 * x.numel() * 2 + C * 2, \
            "F.rms_norm bf16 (4096, 4096) = 1/4 of the workload"

    def ln_cpu():
        x, w, b = norm_cpu_inputs()
        return (lambda: F.layer_norm(x, (C,), w, b, 1e-5)), 2 * x.numel() * 2 + 2 * C * 2, \
            "F.layer_norm bf16 (4096, 4096) = 1/4 of the workload"

    W.append(Workload("rms_norm", "rms_norm bf16 (16384, 4096), weight (4096,), eps 1e-6", "GB/s", "hbm",
                      2 * R * C * 2 + C * 2, 1, norm_build, rms_step, rms_cpu, "bf16"))
    W.append(Workload("layer_norm", "layer_norm bf16 (16384, 4096), weight + bias (4096,), eps 1e-5", "GB/s",
                      "hbm", 2 * R * C * 2 + 2 * C * 2, 1, norm_build, ln_step, ln_cpu, "bf16"))

    # the same norms on rows the register-resident kernels do not take:
    # an odd width (16384, 4100) -- head / packs / tail, parameters in LDS --
    # and wide rows (512, 131072) staged in VGPRs + LDS (rms_norm, softmax)
    RO, CO = 16384, 4100
    RW, CW = 512, 131072

    def odd_build(i):
        g = _gen(120 + i)
        x = torch.randn(RO, CO, device="cuda", generator=g).bfloat16()
        w = (1 + 0.02 * torch.randn(CO, device="cuda", generator=g)).bfloat16()
        return {"x": x, "w": w, "y": torch.empty_like(x)}

    def rms_odd_step(s):
        check(lib.ntops_rms_norm(_lib.BF16, RO, CO, s["x"].data_ptr(), CO, s["w"].data_ptr(), 0, _lib.BF16, 1e-6,
                                 s["y"].data_ptr(), CO, stream()), "rms_norm")

    def wide_build(i):
        g = _gen(140 + i)
        x = torch.randn(RW, CW, device="cuda", generator=g).bfloat16()
        w = (1 + 0.02 * torch.randn(CW, device="cuda", generator=g)).bfloat16()
        return {"x": x, "w": w, "y": torch.empty_like(x)}

    def rms_wide_step(s):
        check(lib.ntops_rms_norm(_lib.BF16, RW, CW, s["x"].data_ptr(), CW, s["w"].data_ptr(), 0, _lib.BF16, 1e-6,
                                 s["y"].data_ptr(), CW, stream()), "rms_norm")

    wide_strides = _lib.i64_array((CW, 1, 1))

    def sm_wide_step(s):
        check(lib.ntops_softmax(_lib.BF16, _lib.BF16, RW, CW, 1, s["x"].data_ptr(), wide_strides, s["y"].data_ptr(),
                                wide_strides, stream()), "softmax")

    W.append(Workload("rms_norm_odd", "rms_norm bf16 (16384, 4100), weight (4100,), eps 1e-6 (rows not 16-byte runs)",
                      "GB/s", "hbm", 2 * RO * CO * 2 + CO * 2, 1, odd_build, rms_odd_step, None, "bf16"))
    W[-1].yardstick = (lambda s: F.rms_norm(s["x"], (CO,), s["w"], 1e-6), "torch rms_norm (GPU), eager")
    W.append(Workload("rms_norm_wide", "rms_norm bf16 (512, 131072), weight (131072,), eps 1e-6 (rows staged in LDS)",
                      "GB/s", "hbm", 2 * RW * CW * 2 + CW * 2, 1, wide_build, rms_wide_step, None, "bf16"))
    W[-1].yardstick = (lambda s: F.rms_norm(s["x"], (CW,), s["w"], 1e-6), "torch rms_norm (GPU), eager")
    W.append(Workload("softmax_wide", "softmax bf16 (512, 131072) dim=-1 (rows staged in LDS)", "GB/s", "hbm",
                      2 * RW * CW * 2, 1, wide_build, sm_wide_step, None, "bf16"))
    W[-1].yardstick = (lambda s: torch.softmax(s["x"], -1), "torch softmax (GPU), eager")

    # softmax bf16 (4, 32, 2048, 2048) causal
    SB, SH, SS = 4, 32, 2048

    def sm_build(i):
        g = _gen(200 + i)
        mask = torch.triu(torch.ones(SS, SS, dtype=torch.bool, device="cuda"), 1)
        x = torch.empty(SB, SH, SS, SS, dtype=torch.bfloat16, device="cuda")
        for b in range(SB):
            x[b] = (torch.randn(SH, SS, SS, device="cuda", generator=g) / math.sqrt(128)).masked_fill(
                mask, float("-inf")).bfloat16()
        return {"x": x, "y": torch.empty_like(x)}

    sm_strides = _lib.i64_array((SS, 1, 1))

    def sm_step(s):
        check(lib.ntops_softmax(_lib.BF16, _lib.BF16, SB * SH * SS, SS, 1, s["x"].data_ptr(), sm_strides,
                                s["y"].data_ptr(), sm_strides, stream()), "softmax")

    def sm_cpu():
        g = _cpu_gen()
        mask = torch.triu(torch.ones(SS, SS, dtype=torch.bool), 1)
        x = (torch.randn(1, 4, SS, SS, generator=g) / math.sqrt(128)).masked_fill(mask, float("-inf")).bfloat16()
        return (lambda: F.softmax(x, -1)), 2 * x.numel() * 2, "F.softmax bf16 (1, 4, 2048, 2048) = 1/32 of the workload"

    W.append(Workload("softmax", "softmax bf16 (4, 32, 2048, 2048) dim=-1, causal -inf mask", "GB/s", "hbm",
                      2 * SB * SH * SS * SS * 2, 1, sm_build, sm_step, sm_cpu, "bf16"))

    # RoPE bf16 q and k (4, 4096, 32, 128), tables (4096, 128)
    RB, RS, RH, RD = 4, 4096, 32, 128
    # tables: theta_i = 10000^(-2i/128), positions 0..4095, built in fp32,
    # duplicated to (4096, 128) (rotate_half convention), cast to bf16
    theta = 10000.0 ** (-2 * (torch.arange(RD // 2, dtype=torch.float32) / RD))
    ang = torch.arange(RS, dtype=torch.float32)[:, None] * theta[None, :]
    sn = torch.cat([torch.sin(ang), torch.sin(ang)], -1)
    cs = torch.cat([torch.cos(ang), torch.cos(ang)], -1)
    sin_t = sn.bfloat16().cuda()
    cos_t = cs.bfloat16().cuda()

    def rope_build(i):
        g = _gen(300 + i)
        q = torch.randn(RB, RS, RH, RD, device="cuda", generator=g).bfloat16()
        k = torch.randn(RB, RS, RH, RD, device="cuda", generator=g).bfloat16()
        return {"q": q, "k": k, "qo": torch.empty_like(q), "ko": torch.empty_like(k),
                "st": _lib.i64_array(q.stride())}

    def rope_step(s):
        for x, y in ((s["q"], s["qo"]), (s["k"], s["ko"])):
            check(lib.ntops_rope(_lib.BF16, RB, RS, RH, RD, x.data_ptr(), s["st"], sin_t.data_ptr(),
                                 cos_t.data_ptr(), RD, RD, 0, y.data_ptr(), s["st"], stream()), "rope")

    def rope_cpu():
        g = _cpu_gen()
        q = torch.randn(1, RS, RH, RD, generator=g).bfloat16()
        st, ct = sn.bfloat16(), cs.bfloat16()

        def run():
            rot = torch.cat((-q[..., RD // 2:], q[..., : RD // 2]), -1)
            return q * ct[None, :, None, :] + rot * st[None, :, None, :]

        return run, 2 * q.numel() * 2 + 2 * RS * RD * 2, \
            "torch eager x*cos + rotate_half(x)*sin, bf16 q (1, 4096, 32, 128) = 1/8 of the workload"

    W.append(Workload("rope", "rotary_position_embedding bf16 q and k (4, 4096, 32, 128), (4096, 128) tables, "
                      "non-interleaved", "GB/s", "hbm", 2 * (2 * RB * RS * RH * RD * 2 + 2 * RS * RD * 2), 2,
                      rope_build, rope_step, rope_cpu, "bf16"))

    # the same q and k rotated in one launch (tables read once)
    def rope_qk_step(s):
        check(lib.ntops_rope_qk(_lib.BF16, RB, RS, RH, RH, RD, s["q"].data_ptr(), s["st"], s["k"].data_ptr(),
                                s["st"], sin_t.data_ptr(), cos_t.data_ptr(), RD, RD, 0, s["qo"].data_ptr(), s["st"],
                                s["ko"].data_ptr(), s["st"], stream()), "rope_qk")

    def rope_qk_cpu():
        run, work, sample = rope_cpu()
        return run, work, sample + " (q and k cost the same)"

    W.append(Workload("rope_qk", "rotary_position_embedding_qk bf16 q and k (4, 4096, 32, 128) in one launch, "
                      "(4096, 128) tables, non-interleaved", "GB/s", "hbm",
                      2 * 2 * RB * RS * RH * RD * 2 + 2 * RS * RD * 2, 1, rope_build, rope_qk_step, rope_qk_cpu,
                      "bf16"))

    # residual add + rms_norm bf16 (16384, 4096): reads x and the residual,
    # writes the new residual and the output
    def arn_build(i):
        s = norm_build(i)
        s["r"] = torch.randn(R, C, device="cuda", generator=_gen(150 + i)).bfloat16()
        s["ro"] = torch.empty_like(s["x"])
        return s

    def arn_step(s):
        check(lib.ntops_add_rms_norm(_lib.BF16, R, C, s["x"].data_ptr(), C, s["r"].data_ptr(), C, s["w"].data_ptr(),
                                     0, _lib.BF16, 1e-6, s["y"].data_ptr(), C, s["ro"].data_ptr(), C, stream()),
              "add_rms_norm")

    def arn_cpu():
        x, w, _ = norm_cpu_inputs()
        r = torch.randn(x.shape, generator=_cpu_gen(1)).bfloat16()

        def run():
            h = x + r
            return F.rms_norm(h, (C,), w, 1e-6), h

        return run, 4 * x.numel() * 2 + C * 2, "torch x + residual then F.rms_norm, bf16 (4096, 4096) = 1/4 of the workload"

    W.append(Workload("add_rms_norm", "add_rms_norm bf16 (16384, 4096): new residual = x + residual, "
                      "rms_norm(new residual) * weight, eps 1e-6", "GB/s", "hbm", 4 * R * C * 2 + C * 2, 1,
                      arn_build, arn_step, arn_cpu, "bf16"))

    # GEMMs
    M, N, K = 8192, 14336, 4096

    def mm_build(i):
        g = _gen(400 + i)
        a = (0.02 * torch.randn(M, K, device="cuda", generator=g)).bfloat16()
        b = (0.02 * torch.randn(K, N, device="cuda", generator=g)).bfloat16()
        bias = (0.02 * torch.randn(N, device="cuda", generator=g)).bfloat16()
        return {"a": a, "b": b, "bias": bias.expand(M, N), "bias1": bias,
                "out": torch.empty(M, N, dtype=torch.bfloat16, device="cuda")}

    def mm_step(s):
        gemm(s["a"], s["b"], s["out"])

    def addmm_step(s):
        gemm(s["a"], s["b"], s["out"], c=s["bias"], alpha=1.0, beta=1.0)

    def mm_cpu_inputs():
        g = _cpu_gen()
        a = (0.02 * torch.randn(512, K, generator=g)).bfloat16()
        b = (0.02 * torch.randn(K, N, generator=g)).bfloat16()
        bias = (0.02 * torch.randn(N, generator=g)).bfloat16()
        return a, b, bias

    def mm_cpu():
        a, b, _ = mm_cpu_inputs()
        return (lambda: torch.mm(a, b)), 2 * 512 * K * N, "torch.mm bf16 (512 x 4096).(4096 x 14336) = 1/16 of the workload"

    def addmm_cpu():
        a, b, bias = mm_cpu_inputs()
        return (lambda: torch.addmm(bias, a, b)), 2 * 512 * K * N, \
            "torch.addmm bf16 bias + (512 x 4096).(4096 x 14336) = 1/16 of the workload"

    W.append(Workload("mm", "mm bf16 (8192 x 4096).(4096 x 14336), fp32 accumulate", "TFLOP/s", "mfma",
                      2 * M * N * K, 1, mm_build, mm_step, mm_cpu, "bf16"))
    W[-1].bytes = (M * K + K * N + M * N) * 2
    W[-1].yardstick = (lambda s: torch.mm(s["a"], s["b"], out=s["out"]), "torch.mm (hipBLASLt), eager")
    W.append(Workload("addmm", "addmm bf16 bias (14336,) + (8192 x 4096).(4096 x 14336), beta = alpha = 1",
                      "TFLOP/s", "mfma", 2 * M * N * K, 1, mm_build, addmm_step, addmm_cpu, "bf16"))
    W[-1].bytes = (M * K + K * N + M * N + N) * 2
    W[-1].yardstick = (lambda s: torch.addmm(s["bias1"], s["a"], s["b"], out=s["out"]),
                       "torch.addmm (hipBLASLt), eager")

    BB, BM, BK, BN = 32, 2048, 128, 2048

    def bmm_build(i):
        g = _gen(500 + i)
        a = (0.02 * torch.randn(BB, BM, BK, device="cuda", generator=g)).bfloat16()
        b = (0.02 * torch.randn(BB, BK, BN, device="cuda", generator=g)).bfloat16()
        return {"a": a, "b": b, "out": torch.empty(BB, BM, BN, dtype=torch.bfloat16, device="cuda")}

    def bmm_step(s):
        gemm(s["a"], s["b"], s["out"], what="bmm")

    def bmm_cpu():
        g = _cpu_gen()
        a = (0.02 * torch.randn(4, BM, BK, generator=g)).bfloat16()
        b = (0.02 * torch.randn(4, BK, BN, generator=g)).bfloat16()
        return (lambda: torch.bmm(a, b)), (4 * BM * BK + 4 * BK * BN + 4 * BM * BN) * 2, \
            "torch.bmm bf16 4 x (2048 x 128).(128 x 2048) = 1/8 of the workload"

    # bmm is HBM-bound (114 flop/B < ridge): judged on bytes
    W.append(Workload("bmm", "bmm bf16 32 x (2048 x 128).(128 x 2048), fp32 accumulate", "GB/s", "hbm",
                      (BB * BM * BK + BB * BK * BN + BB * BM * BN) * 2, 1, bmm_build, bmm_step, bmm_cpu, "bf16"))
    W[-1].flops = 2 * BB * BM * BN * BK
    W[-1].yardstick = (lambda s: torch.bmm(s["a"], s["b"], out=s["out"]), "torch.bmm (hipBLASLt), eager")

    # scaled_dot_product_attention bf16 causal, (4, 32, 2048, 128): the
    # algorithmic flops are those of the unmasked (q, kv) pairs, S (S + 1) / 2
    # per head, each costing 2 D for Q K^T and 2 D for P V
    AB, AH, AS, AD = 4, 32, 2048, 128
    sdpa = ntops_amd.torch.scaled_dot_product_attention

    def sdpa_build(i):
        g = _gen(600 + i)
        q, k, v = (torch.randn(AB, AH, AS, AD, device="cuda", generator=g).bfloat16() for _ in range(3))
        return {"q": q, "k": k, "v": v}

    def sdpa_step(s):
        sdpa(s["q"], s["k"], s["v"], is_causal=True)

    def sdpa_cpu():
        g = _cpu_gen()
        q, k, v = (torch.randn(AB, AH, AS, AD, generator=g).bfloat16() for _ in range(3))
        return (lambda: F.scaled_dot_product_attention(q, k, v, is_causal=True)), \
            4 * AB * AH * AD * AS * (AS + 1) // 2, \
            "torch scaled_dot_product_attention bf16 causal (4, 32, 2048, 128) = the whole workload"

    W.append(Workload("sdpa", "scaled_dot_product_attention bf16 causal (4, 32, 2048, 128), fp32 softmax",
                      "TFLOP/s", "mfma", 4 * AB * AH * AD * AS * (AS + 1) // 2, 1, sdpa_build, sdpa_step,
                      sdpa_cpu, "bf16"))
    W[-1].bytes = 4 * AB * AH * AS * AD * 2

    def sdpa_torch(s):
        # flash / memory-efficient backends only, a precaution: torch's math
        # backend would compute Q K^T as a bf16 batched product over a
        # transposed view, a call documented to fault MI355X GPUs under this
        # torch / ROCm build; restricted, torch raises instead of falling back
        from torch.nn.attention import SDPBackend, sdpa_kernel
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            F.scaled_dot_product_attention(s["q"], s["k"], s["v"], is_causal=True)

    W[-1].yardstick = (sdpa_torch, "torch scaled_dot_product_attention (flash / memory-efficient backend), eager")

    # conv2d bf16 (32, 256, 56, 56) * (256, 256, 3, 3), padding 1: one call
    # is the weight reorder and the zero-padded channels-last copy of the
    # input into the workspace, then the implicit-GEMM matrix-core kernel
    CN, CC, CH, CK = 32, 256, 56, 256
    conv = ntops_amd.torch.conv2d

    def conv_build(i):
        g = _gen(700 + i)
        x = torch.randn(CN, CC, CH, CH, device="cuda", generator=g).bfloat16()
        w = (torch.randn(CK, CC, 3, 3, device="cuda", generator=g) / 48).bfloat16()
        b = torch.randn(CK, device="cuda", generator=g).bfloat16()
        return {"x": x, "w": w, "b": b}

    def conv_step(s):
        conv(s["x"], s["w"], s["b"], padding=1)

    def conv_cpu():
        g = _cpu_gen()
        x = torch.randn(2, CC, CH, CH, generator=g).bfloat16()
        w = (torch.randn(CK, CC, 3, 3, generator=g) / 48).bfloat16()
        b = torch.randn(CK, generator=g).bfloat16()
        return (lambda: F.conv2d(x, w, b, padding=1)), 2 * 2 * CK * CC * 9 * CH * CH, \
            "torch conv2d bf16 (2, 256, 56, 56) * (256, 256, 3, 3) = 1/16 of the workload"

    # im2col bf16 (32, 256, 56, 56), 3x3, padding 1: the conv workload's
    # unfold as the public op (reads the input once, writes 9x it)
    i2c = ntops_amd.torch.im2col

    def i2c_step(s):
        i2c(s["x"], 3, padding=1)

    def i2c_cpu():
        x = torch.randn(2, CC, CH, CH, generator=_cpu_gen()).bfloat16()
        return (lambda: F.unfold(x, 3, padding=1)), 2 * (x.numel() + 2 * CC * 9 * CH * CH), \
            "F.unfold bf16 (2, 256, 56, 56), 3x3, padding 1 = 1/16 of the workload"

    W.append(Workload("im2col", "im2col bf16 (32, 256, 56, 56), kernel 3x3, padding 1 -> (32, 2304, 3136)", "GB/s",
                      "hbm", 2 * (CN * CC * CH * CH + CN * CC * 9 * CH * CH), 1, conv_build, i2c_step, i2c_cpu, "bf16"))

    W.append(Workload("conv2d", "conv2d bf16 (32, 256, 56, 56) * (256, 256, 3, 3) + bias, padding 1 "
                      "(channels-last copy + implicit-GEMM MFMA)", "TFLOP/s", "mfma", 2 * CN * CK * CC * 9 * CH * CH,
                      1, conv_build, conv_step, conv_cpu, "bf16"))
    W[-1].bytes = (2 * CN * CC * CH * CH + CK * CC * 9 + CK) * 2
    W[-1].yardstick = (lambda s: F.conv2d(s["x"], s["w"], s["b"], padding=1), "torch conv2d (MIOpen), NCHW, eager")
    return {w.name: w for w in W}


# -------------------------------------------------------------- timing ----


def settle(run_once, settle_ms):
    """Runs `run_once` (untimed) until `settle_ms` of wall time has passed, so
    the timed runs start with the part's clocks settled for this load."""
    t_end = time.perf_counter() + settle_ms / 1e3
    while True:
        run_once()
        torch.cuda.synchronize()
        if time.perf_counter() >= t_end:
            return


def time_gpu(w, steps, warmup, eager, replays, settle_ms=0.0):
    """Per-step milliseconds of each of `replays` timed runs of `steps` steps
    (a captured K-step graph replayed back to back, or eager launches), after
    `warmup` eager steps and `settle_ms` of untimed runs of the same steps."""
    sets = [w.build(i) for i in range(NSETS)]
    torch.cuda.synchronize()
    for i in range(max(1, warmup)):  # >= 1: one-time kernel attributes are set outside capture
        w.step(sets[i % NSETS])
    torch.cuda.synchronize()
    events = [torch.cuda.Event(enable_timing=True) for _ in range(replays + 1)]

    def eager_steps():
        for i in range(steps):
            w.step(sets[i % NSETS])

    if eager:
        settle(eager_steps, settle_ms)
        events[0].record()
        for r in range(replays):
            for i in range(steps):
                w.step(sets[i % NSETS])
            events[r + 1].record()
        torch.cuda.synchronize()
    else:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(steps):
                w.step(sets[i % NSETS])
        graph.replay()  # one untimed replay (the graph's first launch)
        torch.cuda.synchronize()
        settle(graph.replay, settle_ms)
        graph.replay()  # keeps the GPU busy while the timed replays are queued
        events[0].record()
        for r in range(replays):
            graph.replay()
            events[r + 1].record()
        torch.cuda.synchronize()
        del graph
    ms = [events[r].elapsed_time(events[r + 1]) / steps for r in range(replays)]
    del sets
    torch.cuda.empty_cache()
    return ms


def time_yardstick(fn, build, steps, replays, settle_ms=0.0):
    """Eager per-step milliseconds (median of `replays` runs of `steps`
    calls over the rotating buffer sets) of a library call, after the same
    settling as the workload's own timing; kept out of graph capture, which
    library calls are not guaranteed to survive."""
    sets = [build(i) for i in range(NSETS)]
    for i in range(3):
        fn(sets[i % NSETS])
    torch.cuda.synchronize()

    def eager_steps():
        for i in range(steps):
            fn(sets[i % NSETS])

    settle(eager_steps, settle_ms)
    events = [torch.cuda.Event(enable_timing=True) for _ in range(replays + 1)]
    events[0].record()
    for r in range(replays):
        for i in range(steps):
            fn(sets[i % NSETS])
        events[r + 1].record()
    torch.cuda.synchronize()
    ms = [events[r].elapsed_time(events[r + 1]) / steps for r in range(replays)]
    del sets
    torch.cuda.empty_cache()
    return statistics.median(ms)


def cpu_threads():
    """Host threads for the CPU baseline: every CPU this process may run on
    (its affinity mask), as the baseline's recipe asks."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, n)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def time_cpu(w):
    fn, work, sample = w.cpu()
    reps = 2 if w.name in ("mm", "addmm") else 3
    fn()  # warmup
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    sec = statistics.median(ts)
    rate = work / sec / (1e12 if w.unit == "TFLOP/s" else 1e9)
    return {"value": round(rate, 3), "unit": w.unit, "cores": torch.get_num_threads(), "affinity_cpus": cpu_threads(),
            "kind": "reference",
            "sample": f"{sample}; PyTorch {torch.__version__} CPU op, median of {reps} after 1 warmup, "
                      f"{cpu_model()}"}


def result_for(w, ms_list, measured_traffic, measured_mfma):
    ms = statistics.median(ms_list)
    sec = ms / 1e3
    if w.unit == "TFLOP/s":
        value = w.work / sec / 1e12
        peak, unit = MFMA_BF16_PEAK_TFLOPS, "TFLOP/s"
    else:
        value = w.work / sec / 1e9
        peak, unit = HBM_PEAK_GBS, "GB/s"
    per_kernel_ms = ms / w.kernels_per_step
    achieved = (w.work / w.kernels_per_step) / (per_kernel_ms / 1e3) / (1e12 if unit == "TFLOP/s" else 1e9)
    out = {
        "workload": w.desc,
        "value": round(value, 3),
        "unit": unit,
        "ms_per_step": round(ms, 5),
        "kernel_ms": round(per_kernel_ms, 5),
        "replay_ms_per_step": [round(m, 5) for m in ms_list],
        "replay_spread": round((max(ms_list) - min(ms_list)) / ms, 4),
        "roofline": {"bound": w.bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
                     "frac": round(achieved / peak, 4), "traffic": None},
    }
    t = measured_traffic.get(w.name)
    if t:
        # HBM bytes per launch measured by rocprofv3 (profiles/traffic.json)
        out["roofline"]["traffic"] = t["bytes"]
        out["roofline"]["algorithmic_bytes_per_launch"] = (
            w.work // w.kernels_per_step if unit == "GB/s" else getattr(w, "bytes", None))
    m = measured_mfma.get(w.name)
    if m:
        # matrix-core busy fraction of the kernel (profiles/mfma.json)
        out["roofline"]["mfma_busy"] = m["busy"]
        out["roofline"]["mfma_flops_per_launch"] = m.get("flops")
    if getattr(w, "flops", None):
        out["tflops"] = round(w.flops / sec / 1e12, 3)
    return out


def load_json_kernels(path):
    try:
        with open(path) as f:
            return json.load(f).get("kernels", {})
    except (OSError, ValueError):
        return {}


def main():
    args = parse_args()
    if args.rocprof_summary:
        rocprof_summary(args.rocprof_summary)
        return
    if args.traffic:
        traffic(args.traffic)
        return
    if args.mfma:
        mfma_report(args.mfma)
        return
    if args.counters:
        counter_table(args.counters, args.kernels)
        return
    if args.gpus != 1:
        print(f"bench.py: this library measures one GPU; --gpus {args.gpus} is not supported "
              "(every op runs on a single MI355X; the ops are not sharded across GPUs)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.replays < 1 or args.steps < 1:
        print("bench.py: --steps and --replays must be >= 1", file=sys.stderr)
        sys.exit(2)
    torch.set_num_threads(cpu_threads())
    measured_traffic = load_traffic(args.traffic_file)
    measured_mfma = load_json_kernels(args.mfma_file)
    workloads = make_workloads()
    names = list(workloads) if args.ops == "all" else args.ops.split(",")
    headline = "rms_norm" if "rms_norm" in names else names[0]
    names = [headline] + [n for n in names if n != headline]

    results = {}
    for n in names:
        w = workloads[n]
        ms = time_gpu(w, args.steps, args.warmup, args.eager, args.replays, args.settle_ms)
        r = result_for(w, ms, measured_traffic, measured_mfma)
        y = getattr(w, "yardstick", None)
        if y is not None:
            fn, lib_desc = y
            try:
                y_ms = time_yardstick(fn, w.build, args.steps, args.replays, args.settle_ms)
            except Exception as e:  # a library backend missing on this install
                r["yardstick"] = {"library": lib_desc, "error": f"{type(e).__name__}: {str(e)[:200]}"}
            else:
                y_val = w.work / (y_ms / 1e3) / (1e12 if w.unit == "TFLOP/s" else 1e9)
                r["yardstick"] = {"library": lib_desc, "ms_per_step": round(y_ms, 5), "value": round(y_val, 3),
                                  "unit": w.unit, "ratio": round(r["value"] / y_val, 4)}
        if not args.no_cpu and w.cpu is not None:
            r["cpu_baseline"] = time_cpu(w)
        results[n] = r
        print(f"# {n}: {r['value']} {r['unit']} ({r['kernel_ms'] * 1e3:.1f} us/kernel, "
              f"{100 * r['roofline']['frac']:.1f}% of roofline, replay spread {100 * r['replay_spread']:.1f}%"
              + (f"; {r['yardstick']['library']}: {r['yardstick'].get('value', 'error')} {w.unit}"
                 if "yardstick" in r else "")
              + ")", file=sys.stderr, flush=True)
    ceiling = mceiling = None
    if "copy" in results:
        # every bandwidth-bound kernel against the measured streaming ceiling
        ceiling = results["copy"]["roofline"]["achieved"]
        for r in results.values():
            if r["unit"] == "GB/s":
                r["roofline"]["frac_of_copy"] = round(r["roofline"]["achieved"] / ceiling, 4)
    if "mfma_ceiling" in results:
        # every matrix-bound kernel against the measured matrix-core rate
        mceiling = results["mfma_ceiling"]["roofline"]["achieved"]
        for n, r in results.items():
            if r["unit"] == "TFLOP/s" and n != "mfma_ceiling":
                r["roofline"]["frac_of_mfma_ceiling"] = round(r["roofline"]["achieved"] / mceiling, 4)

    h = results[headline]
    line = {
        "metric": METRIC,
        "value": h["value"],
        "unit": h["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": h["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": workloads[headline].dtype,
        "data": "synthetic (seeded torch.randn of the configured shapes, resident in HBM)",
        "config": {"workload": h["workload"],
                   "timing": ("eager" if args.eager else "hip-graph of K steps") +
                             f", median of {args.replays} timed replays",
                   "settle_ms": args.settle_ms,
                   "buffer_sets": NSETS},
        "roofline": h["roofline"],
        "cpu_baseline": h.get("cpu_baseline"),
        "hbm_ceiling": None if ceiling is None else {
            "copy_gbs": round(ceiling, 3), "frac_of_peak": round(ceiling / HBM_PEAK_GBS, 4),
            "kernel": "ntops_cast fp32 -> fp32, 128 MiB in + 128 MiB out per step (k_cast_pack)"},
        "mfma_ceiling": None if mceiling is None else {
            "tflops": round(mceiling, 3), "frac_of_peak": round(mceiling / MFMA_BF16_PEAK_TFLOPS, 4),
            "kernel": "ntops_mfma_rate_probe (k_mfma_probe), bf16 32x32x16 MFMAs on register operands"},
        "ops": {n: r for n, r in results.items() if n != headline},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
