"""Benchmark: one MI355X, MoE-layer forward + backward tokens/s on the BASELINE workload.

    python bench.py [--steps K] [--warmup W] [--config C2] [--gpus 1] [--no-cpu-baseline]

A step is one forward + gather-only backward of the whole MoE layer (router top-k, layout, dispatch into 128-row
expert blocks, gate/up GEMM + SiLU*mul, down GEMM, combine + shared expert; backward down to dx, every dW and
dW_r) over T tokens of synthetic bf16 input already resident in HBM.  Prints one JSON line.

roofline: the dominant kernel (largest share of the step, found with HIP events on the launch stream in a short
profiled pass that runs every kernel on one stream) is bracketed by a pair of HIP events in every timed step;
achieved = algorithmic flops (or bytes) per launch / its mean event-timed duration.  The timed region runs the
layer's independent chains on helper streams (--concurrency 1, the default; lsurge_set_concurrency).
cpu_baseline: the numpy CPU oracle's float32 layer forward + backward at the config's full token count, timed on this
host; at C2 also `cpu_baseline_c1_fwd`, the C1 forward (BASELINE.md's pair).

--fp8: every expert GEMM on FP8 operands with current scaling (E4M3 activations and weights, E5M2 gradients:
lsurge_moe_fwd_fp8 + lsurge_moe_bwd_fp8); a step is the weights' quantisation (once per optimizer step in training)
plus the forward and backward (--fwd-only: the forward alone); `ms_per_step_cached_weights` times the same without
the weights' quantisation (as in serving, for --fwd-only).  GEMM rooflines are priced against the fp8 peak.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "lewi-surge_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_FP8_TFLOPS = 5000.0   # MI355X dense fp8 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
PEAK_FP32_TFLOPS = 157.3   # MI355X dense fp32 matrix

CONFIGS = {  # BASELINE.json configs (T, d, E, k, f, fs, zipf bias, fwd+bwd)
    "C1": dict(T=4096, d=1024, E=64, k=6, f=512, fs=512, zipf=False, bwd=False),
    "C2": dict(T=16384, d=1024, E=64, k=6, f=512, fs=512, zipf=False, bwd=True),
    "C3": dict(T=16384, d=1024, E=128, k=6, f=512, fs=512, zipf=False, bwd=True),
    "C4": dict(T=32768, d=1024, E=128, k=6, f=512, fs=512, zipf=True, bwd=True),
    "C5": dict(T=65536, d=2048, E=256, k=8, f=512, fs=2048, zipf=False, bwd=True),
}


def fused_router(c):
    """Shapes whose router runs as one kernel (logits, top-k, softmax, the layout's per-64-token histograms)."""
    return c["E"] in (32, 64, 128, 256) and c["k"] <= 8 and c["d"] % 64 == 0


def kernel_work(c, fp8=False):
    """Algorithmic work per launch of each kernel: ('mfma', flops) over useful rows, or ('hbm', bytes)."""
    T, d, E, k, f, fs = c["T"], c["d"], c["E"], c["k"], c["f"], c["fs"]
    M = T * k
    # the bf16 backward's grouped GEMMs carry the shared expert as one more expert (T rows) when fs == f; the FP8
    # backward runs it as dense GEMMs of its own
    merged = bool(fs) and fs == f and not fp8
    Mb = M + T if merged else M
    w = {
        "gemm_gu_fwd": ("mfma", 2 * M * d * 2 * f),
        "gemm_down_fwd": ("mfma", 2 * M * f * d),
        "gemm_down_dgrad": ("mfma", 2 * Mb * d * f),
        "gemm_down_wgrad": ("mfma", 2 * Mb * f * d),
        "gemm_gu_dgrad": ("mfma", 2 * Mb * 2 * f * d),
        "gemm_gu_wgrad": ("mfma", 2 * Mb * d * 2 * f),
        "router_wgrad": ("mfma", 2 * T * d * E),
        "router_topk": ("hbm", T * d * 2 + d * E * 2 + T * E * 4
                        + (8 * T * k + 4 * E * ((T + 63) // 64) if fused_router(c) else 0)),
        "router_select": ("hbm", T * E * 4 + 8 * T * k),
        "dispatch": ("hbm", 2 * M * d * 2 + 4 * M),
        "combine_fwd": ("hbm", M * d * 2 + T * d * 2 * (2 if fs else 1) + 8 * T * k),
        "combine_bwd": ("hbm", 2 * M * d * 2 + T * d * 2 * (2 if Mb > M else 1) + 16 * T * k),  # + dY copy
        "dispatch_bwd": ("hbm", M * d * 2 + T * d * 2 * (2 if fs else 1) + 12 * T * k),
        "layout_hist": ("hbm", 4 * M),
        "layout_rank": ("hbm", 4 * M + 16 * M),
    }
    if fs:
        w.update({
            "shared_gu_fwd": ("mfma", 2 * T * d * 2 * fs),
            "shared_down_fwd": ("mfma", 2 * T * fs * d),
        })
    if fs and not merged:
        w.update({
            "shared_down_dgrad": ("mfma", 2 * T * d * fs),
            "shared_down_wgrad": ("mfma", 2 * T * fs * d),
            "shared_gu_dgrad": ("mfma", 2 * T * 2 * fs * d),
            "shared_gu_wgrad": ("mfma", 2 * T * d * 2 * fs),
        })
    return w


def layer_flops(c):
    """Useful flops of one step: 6 M d f + 6 T d fs + 2 T d E per forward, x3 for forward + backward."""
    T, d, E, k, f, fs = c["T"], c["d"], c["E"], c["k"], c["f"], c["fs"]
    fwd = 6 * T * k * d * f + 6 * T * d * fs + 2 * T * d * E
    return fwd * (3 if c["bwd"] else 1)


def make_params(c, dev, seed=0):
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)

    def nrm(shape, std):
        return (torch.randn(shape, device=dev, generator=g) * std).to(torch.bfloat16)

    T, d, E, f, fs = c["T"], c["d"], c["E"], c["f"], c["fs"]
    p = dict(x=nrm((T, d), 1.0), w_r=nrm((d, E), 0.02), w_gate=nrm((E, d, f), 0.02), w_up=nrm((E, d, f), 0.02),
             w_down=nrm((E, f, d), 0.02), ws_gate=nrm((d, fs), 0.02) if fs else None,
             ws_up=nrm((d, fs), 0.02) if fs else None, ws_down=nrm((fs, d), 0.02) if fs else None, bias=None)
    if c["zipf"]:
        import math
        p["bias"] = torch.tensor([1.5 * math.log(1.0 / (e + 1)) for e in range(E)], dtype=torch.float32, device=dev)
    dy = nrm((T, d), 1.0)
    return p, dy


def measured_traffic(config, kernel, fp8=False, bwd=True):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (lines
    `bench-traffic <kernel> <bytes>` in profiles/moe_layer_<config>_fwd_bwd.md, or _fp8_fwd_bwd.md / _fp8_fwd.md for
    --fp8), or None."""
    name = ("fp8_fwd_bwd" if bwd else "fp8_fwd") if fp8 else "fwd_bwd"
    return traffic_from(os.path.join(ROOT, "profiles", f"moe_layer_{config.lower()}_{name}.md"), kernel)


def traffic_from(path, kernel):
    """The `bench-traffic <kernel> <bytes>` line of a committed profile summary, or None."""
    try:
        with open(path) as fh:
            for line in fh:
                f = line.split()
                if len(f) == 3 and f[0] == "bench-traffic" and f[1] == kernel:
                    return float(f[2])
    except OSError:
        return None
    return None


def prof_table(lib, steps):
    import ctypes
    out = {}
    for i in range(lib.lsurge_prof_kernel_count()):
        tot, cnt = ctypes.c_double(), ctypes.c_int64()
        lib.lsurge_prof_read(i, ctypes.byref(tot), ctypes.byref(cnt))
        if cnt.value:
            out[lib.lsurge_prof_kernel_name(i).decode()] = (tot.value / cnt.value, cnt.value, tot.value / steps)
    return out


def cpu_baseline(c, target_s=12.0, max_iters=50):
    """Time the numpy oracle (float32) of the same layer at the config's full token count on this host's cores:
    router (the bit-exact C restatement, one thread), forward, and the backward when the config has one.  One warm-up
    call, then calls until target_s has passed (at least one).  Returns the cpu_baseline object of the JSON line."""
    import numpy as np
    from oracle import c_oracle as co
    from oracle import moe_oracle as mo

    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    cores = len(os.sched_getaffinity(0))
    T = c["T"]
    p = mo.make_inputs(T=T, d=c["d"], E=c["E"], k=c["k"], f=c["f"], fs=c["fs"], seed=0, zipf=c["zipf"])
    ctx = threadpool_limits(limits=cores) if threadpool_limits else None
    try:
        def one():
            logits, sel, _ = co.router(p["x"], p["w_r"], p["k"], p.get("bias"))
            out, cache = mo.moe_layer_fwd(p, np.float32, route=(logits, sel))
            if c["bwd"]:
                mo.moe_layer_bwd(p, cache, p["dy"], np.float32)

        one()  # warm-up
        n, t0 = 0, time.perf_counter()
        while True:
            one()
            n += 1
            el = time.perf_counter() - t0
            if el > target_s or n >= max_iters:
                break
    finally:
        if ctx is not None:
            ctx.__exit__(None, None, None)
    return dict(value=T * n / el, unit="tokens/s", cores=cores, kind="port",
                sample=f"numpy float32 oracle ({'fwd+bwd' if c['bwd'] else 'fwd'}) of the same layer at the full T={T} "
                       f"(about {T * c['k'] // c['E']} rows per expert), {n} calls after one warm-up ({el:.1f} s), "
                       f"BLAS threads={cores}, router in C (1 thread)")


# ------------------------------------------------------------------------------------------ profile summary
def short_kernel(name):
    """rocprofv3 kernel name -> template name with its integer template arguments, e.g. gemm_rows_kernel<1,1>."""
    import re
    n = name.replace("void ", "")
    n = re.sub(r"\([^()]*\)$", "", n)               # argument list
    n = re.sub(r"lsgemm::GemmCfg<[^>]*>,? ?", "", n)  # the tile shape (one for every GEMM)
    n = n.replace("lsgemm::", "").replace("(anonymous namespace)::", "")
    n = n.replace(" ", "").replace("<>", "")
    # the GEMM templates' element-type / FP8 flags (defaults) are not part of the role: B layout and epilogue only
    m = re.match(r"(gemm_rows_kernel)<(\d+),(\d+)(,.*)?>$", n)
    if m:
        f8 = m.group(4).strip(",").split(",")[0] if m.group(4) else "0"  # the FP8 flag: 0, or the A format + 1
        n = f"{m.group(1)}<{m.group(2)},{m.group(3)}>" + ("<f8>" if f8 not in ("0", "false") else "")
    if n.startswith("gemm_wgrad_kernel<"):
        n = "gemm_wgrad_kernel"
    # the persistent 256 x 256 kernels: B layout, epilogue and row gather (rows), row gather (weight gradient)
    m = re.match(r"g256::rows_kernel<(\d+),(\d+),(true|false)", n)
    if m:
        n = f"g256_rows<{m.group(1)},{m.group(2)},{int(m.group(3) == 'true')}>"
    m = re.match(r"g256::wgrad_kernel<(true|false)", n)
    if m:
        n = f"g256_wgrad<{int(m.group(1) == 'true')}>"
    return n


def launch_roles(c):
    """Role of every hot-path launch of one layer call, per kernel template, in host submission order."""
    fs, f = c["fs"], c["f"]
    own = bool(fs) and fs != f  # shared expert of its own width: dense backward GEMMs on a helper stream
    r = {
        "router_logits_kernel": ["router_topk"], "router_fused_kernel<64,2>": ["router_topk"],
        "router_fused_kernel<128,4>": ["router_topk"], "router_fused_kernel<256,4>": ["router_topk"],
        "router_select_lane_kernel<8>": ["router_select"],
        "router_select_lane_kernel<16>": ["router_select"], "router_select_kernel<1>": ["router_select"],
        "router_select_kernel<2>": ["router_select"], "router_select_kernel<4>": ["router_select"],
        "layout_hist_kernel": ["layout_hist"], "layout_scan_kernel": ["layout_scan"],
        "layout_rank_kernel": ["layout_rank"], "layout_fused_kernel": ["layout_rank"],
        "gemm_rows_kernel<1,1>": (["shared_gu_fwd"] if fs else []) + ["gemm_gu_fwd"],
        "gemm_rows_kernel<1,0>": (["shared_down_fwd"] if fs else []) + ["gemm_down_fwd"],
        "combine_pad_kernel<2,6,1>": ["combine_fwd"], "combine_pad_kernel<2,8,1>": ["combine_fwd"],
        "combine_pad_kernel<4,8,1>": ["combine_fwd"],
    }
    # persistent kernels (gemm_variant 1): the shared expert's dense forward is the non-gathered SwiGLU launch
    r.update({"g256_rows<1,1,0>": ["shared_gu_fwd"], "g256_rows<1,1,1>": ["gemm_gu_fwd"],
              "g256_rows<1,0,0>": (["shared_down_fwd"] if fs else []) + ["gemm_down_fwd"]})
    g256 = c.get("gemm_variant", 1) == 1
    if c.get("fp8"):
        # FP8 expert GEMMs (classic kernels): the shared expert runs dense GEMMs of its own in both directions, each
        # template's shared launch submitted before the routed one (the FP8 GEMM templates are tagged <f8>)
        sh = bool(fs)
        r.update({
            "gemm_rows_kernel<0,1><f8>": (["shared_gu_fwd"] if sh else []) + ["gemm_gu_fwd"],
            "gemm_rows_kernel<0,0><f8>": (["shared_down_fwd"] if sh else []) + ["gemm_down_fwd"]
                                          + ((["shared_gu_dgrad"] if sh else []) + ["gemm_gu_dgrad"] if c["bwd"] else []),
            "fp8_cast_kernel<false>": ["fp8_cast"] * 8, "fp8_cast_kernel<true>": ["fp8_cast"] * 8,
            "fp8_amax_kernel": ["fp8_amax"] * 16, "fp8_cast_t_kernel": ["fp8_quantize_weights"] * 16,
        })
        if c["bwd"]:
            r.update({
                "gemm_rows_kernel<0,2><f8>": (["shared_down_dgrad"] if sh else []) + ["gemm_down_dgrad"],
                "gemm_wgrad_f8_kernel<0,1>": (["shared_down_wgrad", "shared_gu_wgrad"] if sh else [])
                                             + ["gemm_down_wgrad", "gemm_gu_wgrad"],
                "gemm_wgrad_kernel": ["router_wgrad"],
                "dy_rows_amax_kernel": ["fp8_amax"], "dy_scale_kernel": ["misc"],
                "splitk_reduce_kernel<4>": ["splitk_reduce"] * 3,
                "wgrad_chunk_reduce_kernel": ["chunk_reduce", "chunk_reduce"],
                "wgrad_chunks_kernel": ["misc"], "transpose_bf16_kernel": ["misc"],
                "combine_bwd_pad_kernel<2,6>": ["combine_bwd"], "combine_bwd_pad_kernel<2,8>": ["combine_bwd"],
                "dispatch_bwd_pad_kernel<2,6>": ["dispatch_bwd"], "dispatch_bwd_pad_kernel<2,8>": ["dispatch_bwd"],
            })
        return r
    if c["bwd"]:
        r.update({
            "g256_rows<0,2,0>": (["shared_down_dgrad"] if own else []) + ["gemm_down_dgrad"],
            "g256_rows<0,0,0>": (["shared_gu_dgrad"] if own else []) + ["gemm_gu_dgrad"],
            "g256_wgrad<1>": ["gemm_gu_wgrad"],
        })
        r.update({
            "gemm_rows_kernel<0,2>": (["shared_down_dgrad"] if own else []) + ["gemm_down_dgrad"],
            "gemm_rows_kernel<0,0>": (["shared_gu_dgrad"] if own else []) + ["gemm_gu_dgrad"],
            "gemm_wgrad_kernel": (["shared_down_wgrad", "shared_gu_wgrad"] if own else [])
                                 + (["gemm_down_wgrad", "router_wgrad"] if g256
                                    else ["gemm_down_wgrad", "router_wgrad", "gemm_gu_wgrad"]),
            "splitk_reduce_kernel": ["splitk_reduce"] * (3 if own else 1),
            "wgrad_chunk_reduce_kernel": ["chunk_reduce", "chunk_reduce"],
            "wgrad_chunks_kernel": ["misc"], "transpose_bf16_kernel": ["misc"], "scatter_dlogits_kernel": ["misc"],
            "combine_bwd_pad_kernel<2,6>": ["combine_bwd"], "combine_bwd_pad_kernel<2,8>": ["combine_bwd"],
            "combine_bwd_pad_kernel<4,8>": ["combine_bwd"],
            "dispatch_bwd_pad_kernel<2,6>": ["dispatch_bwd"], "dispatch_bwd_pad_kernel<2,8>": ["dispatch_bwd"],
            "dispatch_bwd_pad_kernel<4,8>": ["dispatch_bwd"],
        })
    return r


def label_launches(rows, c):
    """rows: dicts with Correlation_Id and Kernel_Name -> list of (role, short name, row) for the hot-path launches.
    The forward's dense shared-expert GEMMs (on a helper stream, 256-row tiles) are told apart from the routed ones
    by their workgroup count; otherwise a layer call starts at each router kernel (fused, or the split path's logits
    kernel) and within it the n-th launch of a template has the n-th role."""
    roles = launch_roles(c)
    T, d, fs = c["T"], c["d"], c["fs"]
    pad8 = lambda n: (n + 7) // 8 * 8  # noqa: E731
    tb = (T + 255) // 256
    shared_wgs = {"gemm_rows_kernel<1,1>": pad8((fs + 127) // 128 * tb), "gemm_rows_kernel<1,0>": pad8((d + 255) // 256 * tb)}

    def wgs(row):
        g = row.get("Grid_Size_X", row.get("Grid_Size"))
        w = row.get("Workgroup_Size_X", row.get("Workgroup_Size"))
        return int(g) // max(1, int(w))

    g256 = c.get("gemm_variant", 1) == 1 and not c.get("fp8")
    out, seen = [], {}
    for row in sorted(rows, key=lambda x: int(x["Correlation_Id"])):
        k = short_kernel(row["Kernel_Name"])
        if k == "router_logits_kernel" or k.startswith("router_fused_kernel"):
            seen = {}
        if g256 and fs and k in ("gemm_rows_kernel<1,1>", "gemm_rows_kernel<1,0>"):
            # with helper streams the shared expert's dense forward runs on the classic kernels beside the router,
            # submitted before the routed GEMMs; its down projection then takes the first persistent <1,0,0> role
            # (a merged shared expert's down projection rides along the routed one: that launch is gemm_down_fwd)
            if k == "gemm_rows_kernel<1,0>" or fs == c["f"]:
                seen["g256_rows<1,0,0>"] = max(seen.get("g256_rows<1,0,0>", 0), 1)
            out.append(("shared_gu_fwd" if k == "gemm_rows_kernel<1,1>" else "shared_down_fwd", k, row))
            continue
        if k not in roles:
            continue
        if fs and k in shared_wgs:  # forward GEMM: shared (dense) or routed
            shared = wgs(row) == shared_wgs[k]
            out.append((roles[k][0 if shared else 1], k, row))
            continue
        i = seen.get(k, 0)
        seen[k] = i + 1
        out.append((roles[k][i] if i < len(roles[k]) else "other", k, row))
    return out


def kernel_traffic(a):
    """Per-kernel HBM bytes per dispatch from rocprofv3 FETCH_SIZE / WRITE_SIZE counter runs of any bench.py mode
    (a.pmc_fetch, a.pmc_write), calibrated on --copy-probe runs (a.copy_fetch, a.copy_write) as in profile_summary;
    kernels keyed by short name (gdn_bchunk_kernel -> gdn_bchunk).  Prints a markdown table and one
    `bench-traffic <kernel> <bytes>` line per kernel (read + write bytes per launch)."""
    import csv
    import glob

    def rows_of(d, kind):
        files = glob.glob(os.path.join(d, f"*{kind}.csv"))
        if not files:
            raise SystemExit(f"kernel traffic: no *{kind}.csv under {d}")
        with open(files[0]) as fh:
            return list(csv.DictReader(fh))

    per = {}
    for name, d, cd in (("FETCH_SIZE", a.pmc_fetch, a.copy_fetch), ("WRITE_SIZE", a.pmc_write, a.copy_write)):
        probe = [r for r in rows_of(cd, "counter_collection") if "copyBuffer" in r["Kernel_Name"]]
        fac = (a.copy_probe_mib << 20) / (sum(float(r["Counter_Value"]) for r in probe) / len(probe) * 1024)
        print(f"calibration {name}: x{fac:.3f} (bytes per KiB-count unit x 1024)")
        for r in rows_of(d, "counter_collection"):
            if r["Counter_Name"] != name:
                continue
            k = short_kernel(r["Kernel_Name"])
            if "at::" in k or "copyBuffer" in k:
                continue
            k = k[:-len("_kernel")] if k.endswith("_kernel") else k
            per.setdefault(k, {}).setdefault(name, []).append(float(r["Counter_Value"]) * 1024 * fac)
    print()
    print("| kernel | dispatches | HBM read MB / launch | HBM write MB / launch |")
    print("|---|---|---|---|")
    for k, v in sorted(per.items()):
        rd, wr = v.get("FETCH_SIZE", []), v.get("WRITE_SIZE", [])
        print(f"| {k} | {len(rd)} | {sum(rd) / max(1, len(rd)) / 1e6:.1f} | {sum(wr) / max(1, len(wr)) / 1e6:.1f} |")
    print()
    for k, v in sorted(per.items()):
        if v.get("FETCH_SIZE") and v.get("WRITE_SIZE"):
            print(f"bench-traffic {k} "
                  f"{sum(v['FETCH_SIZE']) / len(v['FETCH_SIZE']) + sum(v['WRITE_SIZE']) / len(v['WRITE_SIZE']):.0f}")


def stats_summary(d):
    """Plain-text table of a rocprofv3 --stats kernel summary (*kernel_stats.csv under d): tile shapes named
    C128 (4-wave, 128 x 256) and PP256 (ping-pong, 256 x 256), argument lists dropped."""
    import csv
    import glob
    import re
    files = glob.glob(os.path.join(d, "*kernel_stats.csv"))
    if not files:
        raise SystemExit(f"stats summary: no *kernel_stats.csv under {d}")
    with open(files[0]) as fh:
        rows = list(csv.DictReader(fh))
    # the bench's own calibration kernel (lsurge_mfma_rate_probe) is not part of the path: left out, shares rescaled
    rows = [r for r in rows if "mfma_rate_kernel" not in r["Name"]]
    tot = sum(int(r["TotalDurationNs"]) for r in rows) or 1
    print(f"{'kernel':58s} {'calls':>6s} {'avg us':>9s} {'total ms':>9s} {'share':>7s}")
    for r in rows:
        n = r["Name"].replace("void ", "")
        n = re.sub(r"\([^()]*\)$", "", n)
        n = n.replace("lsgemm::GemmCfg<128, 256, 32, 2, 2, 3, 2, 0>", "C128")
        n = n.replace("lsgemm::GemmCfg<256, 256, 32, 2, 4, 3, 1, 1>", "PP256")
        n = n.replace("lsgemm::", "").replace("(anonymous namespace)::", "")
        if "at::" in n:
            n = "torch (synthetic inputs)"
        print(f"{n[:58]:58s} {int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:9.1f} "
              f"{int(r['TotalDurationNs']) / 1e6:9.2f} {100 * int(r['TotalDurationNs']) / tot:6.2f}%")


def profile_summary(a):
    """Markdown summary of rocprofv3 outputs of bench.py runs (kernel trace; FETCH_SIZE / WRITE_SIZE counter runs of
    the layer and of --copy-probe for calibration), with `bench-traffic <role> <bytes>` lines for the roofline."""
    import csv
    import glob

    c = dict(CONFIGS[a.config], gemm_variant=a.gemm_variant, fp8=a.fp8)
    if a.fwd_only:
        c["bwd"] = False

    def rows_of(d, kind):
        files = glob.glob(os.path.join(d, f"*{kind}.csv"))
        if not files:
            raise SystemExit(f"profile summary: no *{kind}.csv under {d}")
        with open(files[0]) as fh:
            return list(csv.DictReader(fh))

    trace = label_launches(rows_of(a.profile_summary, "kernel_trace"), c)
    dur = {}
    for role, k, row in trace:
        dur.setdefault((role, k), []).append((int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3)
    counters = {}
    fac = {}
    for name, d, cd in (("FETCH_SIZE", a.pmc_fetch, a.copy_fetch), ("WRITE_SIZE", a.pmc_write, a.copy_write)):
        if not d:
            continue
        probe = [r for r in rows_of(cd, "counter_collection") if "copyBuffer" in r["Kernel_Name"]] if cd else []
        # the copy probe moves 1 GiB per launch: bytes = KiB counter x 1024 x factor
        fac[name] = (a.copy_probe_mib << 20) / (sum(float(r["Counter_Value"]) for r in probe) / len(probe) * 1024) \
            if probe else 1.0
        for role, k, row in label_launches([r for r in rows_of(d, "counter_collection") if r["Counter_Name"] == name], c):
            counters.setdefault((role, name), []).append(float(row["Counter_Value"]) * 1024 * fac[name])
    total = sum(sum(v) for v in dur.values())
    print("| role | kernel | launches | avg us | share of hot-path GPU time | HBM read MB / launch | "
          "HBM write MB / launch |")
    print("|---|---|---|---|---|---|---|")
    traffic = {}
    for (role, k), v in sorted(dur.items(), key=lambda kv: -sum(kv[1])):
        rd = counters.get((role, "FETCH_SIZE"))
        wr = counters.get((role, "WRITE_SIZE"))
        rmb = sum(rd) / len(rd) if rd else None
        wmb = sum(wr) / len(wr) if wr else None
        if rmb is not None and wmb is not None:
            traffic[role] = rmb + wmb
        fmt = lambda x: "-" if x is None else f"{x / 1e6:.1f}"  # noqa: E731
        print(f"| {role} | `{k}` | {len(v)} | {sum(v) / len(v):.1f} | {100 * sum(v) / total:.1f}% | {fmt(rmb)} | "
              f"{fmt(wmb)} |")
    print()
    if a.pmc_extra:
        counter_table(a, c, rows_of)
        print()
    for n, f in fac.items():
        print(f"calibration {n}: x{f:.3f} (bytes per KiB-count unit x 1024)")
    print()
    for role, b in sorted(traffic.items()):
        print(f"bench-traffic {role} {b:.0f}")


def counter_table(a, c, rows_of):
    """Per-role averages of the rocprofv3 --pmc runs in a.pmc_extra (one directory per pass), with derived rates.
    Counter values are whole-GPU sums per dispatch: GRBM_GUI_ACTIVE adds the 8 XCDs' busy cycles, so the clock is
    GRBM_GUI_ACTIVE / 8 / duration; MFMA util = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 x 1024 SIMDs) (the
    counter adds 32 cycles per 32x32x16 MFMA, so this is achieved flops over the peak at the measured clock); TA / TD
    busy = TA_TA_BUSY_sum / TD_TD_BUSY_sum over (GRBM_GUI_ACTIVE / 8 x 256 CUs); LDS issue wait = SQ_WAIT_INST_LDS /
    SQ_WAVE_CYCLES (the share of wave time spent waiting to issue an LDS instruction)."""
    import collections
    per = collections.defaultdict(lambda: collections.defaultdict(list))
    dur = collections.defaultdict(list)
    for d in a.pmc_extra:
        rows = rows_of(d, "counter_collection")
        disp = {}
        for r in rows:
            e = disp.setdefault(r["Dispatch_Id"], dict(r, ctr={}))
            e["ctr"][r["Counter_Name"]] = e["ctr"].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        for role, k, row in label_launches(list(disp.values()), c):
            dns = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
            for n, v in row["ctr"].items():
                per[role][(d, n)].append((v, dns))
            dur[role].append(dns)

    def avg(role, name):
        vals = [(v, t) for (d, n), lst in per[role].items() if n == name for v, t in lst]
        return (sum(v for v, _ in vals) / len(vals), sum(t for _, t in vals) / len(vals)) if vals else (None, None)

    def grbm(role, name):  # GRBM of the same pass as counter `name`
        for (d, n), lst in per[role].items():
            if n == name:
                g = [v for (d2, n2), l2 in per[role].items() if d2 == d and n2 == "GRBM_GUI_ACTIVE" for v, _ in l2]
                return sum(g) / len(g) / 8 if g else None
        return None

    print("| role | avg us | clock GHz | MFMA util | LDS instrs / launch | LDS bank conflicts | LDS issue wait | "
          "TA busy | TD busy | TD waits on L1 (TCP_PENDING) |")
    print("|---|---|---|---|---|---|---|---|---|---|")
    for role in sorted(dur, key=lambda r: -sum(dur[r])):
        g, t = avg(role, "GRBM_GUI_ACTIVE")
        clk = g / 8 / t if g else None
        mf, _ = avg(role, "SQ_VALU_MFMA_BUSY_CYCLES")
        gm = grbm(role, "SQ_VALU_MFMA_BUSY_CYCLES")
        lds, _ = avg(role, "SQ_INSTS_LDS")
        bc, _ = avg(role, "SQ_LDS_BANK_CONFLICT")
        wl, _ = avg(role, "SQ_WAIT_INST_LDS")
        wc, _ = avg(role, "SQ_WAVE_CYCLES")
        ta, _ = avg(role, "TA_TA_BUSY_sum")
        gt = grbm(role, "TA_TA_BUSY_sum")
        td, _ = avg(role, "TD_TD_BUSY_sum")
        tp, _ = avg(role, "TCP_PENDING_STALL_CYCLES_sum")
        f = lambda x, fmt: "-" if x is None else fmt.format(x)  # noqa: E731
        print(f"| {role} | {sum(dur[role]) / len(dur[role]) / 1e3:.1f} | {f(clk, '{:.2f}')} | "
              f"{f(mf / (gm * 1024) if mf is not None and gm else None, '{:.1%}')} | {f(lds, '{:.3g}')} | "
              f"{f(bc, '{:.3g}')} | {f(wl / wc if wl is not None and wc else None, '{:.1%}')} | "
              f"{f(ta / (gt * 256) if ta is not None and gt else None, '{:.0%}')} | "
              f"{f(td / (gt * 256) if td is not None and gt else None, '{:.0%}')} | "
              f"{f(tp / (gt * 256) if tp is not None and gt else None, '{:.0%}')} |")


def conv_bench(a):
    """Causal depthwise Conv1D at configs/stage1.yml's GDN shape: per_device_batch_size 8, max_target_length 4096,
    kernel 4 over 2 x 4 key heads x 128 + 8 value heads x 128 = 2048 channels.  HBM-bound: algorithmic bytes are
    x read + y written (forward), x and dy read + dx written + the f32 partials of dw (backward)."""
    import torch

    import _lib as L

    B, T, C, K = 8, 4096, 2048, 4
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((B, T, C), device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn((K, C), device=dev, generator=g) * 0.5).to(torch.bfloat16)
    dy = torch.randn((B, T, C), device=dev, generator=g).to(torch.bfloat16)
    y, dx = torch.empty_like(x), torch.empty_like(x)
    dw = torch.empty((K, C), dtype=torch.float32, device=dev)
    lib = L.lib()
    ws = L.workspace(lib.lsurge_causal_conv1d_bwd_workspace_bytes(B, T, C, K), dev)
    st = L.stream(dev)
    fwd = lambda: L.check(lib.lsurge_causal_conv1d(L.ptr(x), L.ptr(w), B, T, C, K, L.ptr(y), st), "conv")  # noqa
    bwd = lambda: L.check(lib.lsurge_causal_conv1d_bwd(L.ptr(x), L.ptr(w), L.ptr(dy), B, T, C, K, L.ptr(dx),  # noqa
                                                       L.ptr(dw), L.ptr(ws), ws.numel(), st), "conv_bwd")
    res = {}
    parts = B * ((T + 63) // 64 + 3) // 4  # dw partial slots (written, then read by the reduction)
    nbytes = {"fwd": 2 * B * T * C * 2 + K * C * 2, "bwd": 3 * B * T * C * 2 + K * C * 2 + 2 * parts * K * C * 4}
    for name, fn in (("fwd", fwd), ("bwd", bwd)):
        for _ in range(a.warmup):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(a.steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / a.steps
        res[name] = (ms, nbytes[name] / (ms * 1e-3) / 1e9)
    ms = res["fwd"][0] + res["bwd"][0]
    gbs = (nbytes["fwd"] + nbytes["bwd"]) / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "causal depthwise Conv1D (GDN block) fwd+bwd GB/s @1 GPU", "value": round(gbs, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16 (f32 accumulation)", "data": "synthetic normals",
        "config": {"workload": f"causal depthwise conv1d B={B} T={T} C={C} K={K} (configs/stage1.yml GDN shape)"},
        "fwd": {"ms": round(res["fwd"][0], 4), "GB/s": round(res["fwd"][1], 1)},
        "bwd": {"ms": round(res["bwd"][0], 4), "GB/s": round(res["bwd"][1], 1)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None}}), flush=True)


def gdn_bench(a):
    """Chunked gated delta rule at configs/stage1.yml's GDN shape: per_device_batch_size 8, max_target_length 4096,
    8 value heads x 128 (keys repeated to the value heads), chunks of 64: the forward, and the training step forward +
    backward (the forward keeps its chunk products and states for the backward, as XLA's autodiff keeps residuals; the
    backward that recomputes them instead, as a remat'd step would, is timed beside it).  Algorithmic flops
    per chunk and head, forward: 2 (2 C^2 Dk + 2 C^2 Dv) chunk-local (S, attn, u, w) + 2 (2 C Dk Dv + C^2 Dv + C Dk Dv)
    scan (q S, w S, attn v_new, the state update); the backward counts twice the forward's (the usual 2x for the
    gradients of every product), so fwd + bwd = 3 x forward, counted in full as the reference's dense products are."""
    import torch

    import _lib as L

    B, T, H, D, C = 8, 4096, 8, 128, 64
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn((B, T, H, D), device=dev, generator=gen).to(torch.bfloat16)
    k = torch.nn.functional.normalize(torch.randn((B, T, H, D), device=dev, generator=gen), dim=-1).to(torch.bfloat16)
    v = torch.randn((B, T, H, D), device=dev, generator=gen).to(torch.bfloat16)
    g = -torch.rand((B, T, H), device=dev, generator=gen) * 0.1
    beta = torch.sigmoid(torch.randn((B, T, H), device=dev, generator=gen)).to(torch.bfloat16)
    do = torch.randn((B, T, H, D), device=dev, generator=gen).to(torch.bfloat16)
    o = torch.empty_like(v)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dg = torch.empty((B, T, H), dtype=torch.float32, device=dev)
    db = torch.empty_like(dg)
    lib = L.lib()
    ws = L.workspace(lib.lsurge_gdn_chunked_workspace_bytes(B, T, H, D, D), dev)
    wsb = L.workspace(lib.lsurge_gdn_chunked_bwd_workspace_bytes(B, T, H, D, D), dev)
    saved = L.workspace(lib.lsurge_gdn_chunked_saved_bytes(B, T, H, D, D), dev)
    wss = L.workspace(lib.lsurge_gdn_chunked_bwd_saved_workspace_bytes(B, T, H, D, D), dev)
    st = L.stream(dev)

    def fwd():
        L.check(lib.lsurge_gdn_chunked_fwd(L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(g), L.ptr(beta), B, T, H, D, D, None,
                                           L.ptr(o), None, L.ptr(ws), ws.numel(), st), "gdn_chunked_fwd")

    def bwd_recompute():
        L.check(lib.lsurge_gdn_chunked_bwd(L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(g), L.ptr(beta), B, T, H, D, D, None,
                                           L.ptr(do), None, L.ptr(dq), L.ptr(dk), L.ptr(dv), L.ptr(dg), L.ptr(db), None,
                                           L.ptr(wsb), wsb.numel(), st), "gdn_chunked_bwd")

    def fwd_save():
        L.check(lib.lsurge_gdn_chunked_fwd_save(L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(g), L.ptr(beta), B, T, H, D, D,
                                                None, L.ptr(o), None, L.ptr(saved), saved.numel(), st),
                "gdn_chunked_fwd_save")

    def bwd():
        L.check(lib.lsurge_gdn_chunked_bwd_saved(L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(beta), B, T, H, D, D, L.ptr(do),
                                                 None, L.ptr(dq), L.ptr(dk), L.ptr(dv), L.ptr(dg), L.ptr(db), None,
                                                 L.ptr(saved), saved.numel(), L.ptr(wss), wss.numel(), st),
                "gdn_chunked_bwd_saved")

    def step():
        fwd_save()
        bwd()

    def step_recompute():
        fwd()
        bwd_recompute()

    # per-kernel averages over a few training steps (forward keeping its residuals + backward from them), each
    # launch bracketed by the library's profiler
    for _ in range(2):
        step()
    torch.cuda.synchronize()
    lib.lsurge_prof_reset()
    lib.lsurge_prof_enable(-1)
    for _ in range(3):
        step()
    torch.cuda.synchronize()
    lib.lsurge_prof_collect()
    lib.lsurge_prof_enable(0)
    table = prof_table(lib, 3)
    chunks = B * H * ((T + C - 1) // C)
    kbytes = gdn_kernel_bytes(C, D)
    prof_md = os.path.join(ROOT, "profiles", "gdn_chunked_fwd_bwd.md")
    kern = {}
    for n, (rd, wr) in kbytes.items():
        if n not in table:
            continue
        ms_k = table[n][0]
        kern[n] = {"ms": round(ms_k, 4), "algorithmic_MB": round(chunks * (rd + wr) / 1e6, 1),
                   "GB/s": round(chunks * (rd + wr) / (ms_k * 1e-3) / 1e9, 1),
                   "hbm_frac": round(chunks * (rd + wr) / (ms_k * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                   "traffic": traffic_from(prof_md, n)}
    dom = max(kern, key=lambda n: kern[n]["ms"])
    # the dominant kernel alone bracketed (its launch stream is torch's current one) over a.steps training steps
    names = [lib.lsurge_prof_kernel_name(i).decode() for i in range(lib.lsurge_prof_kernel_count())]
    lib.lsurge_prof_reset()
    lib.lsurge_prof_enable(1 << names.index(dom))
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    lib.lsurge_prof_collect()
    lib.lsurge_prof_enable(0)
    ms_k = prof_table(lib, a.steps)[dom][0]
    rd, wr = kbytes[dom]
    kern[dom].update({"ms": round(ms_k, 4), "GB/s": round(chunks * (rd + wr) / (ms_k * 1e-3) / 1e9, 1),
                      "hbm_frac": round(chunks * (rd + wr) / (ms_k * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)})

    ms_f = _time_ms(fwd, a.steps, a.warmup)
    ms_fs = _time_ms(fwd_save, a.steps, a.warmup)
    ms_b = _time_ms(bwd, a.steps, a.warmup)
    ms_br = _time_ms(bwd_recompute, a.steps, a.warmup)
    ms_r = _time_ms(step_recompute, a.steps, a.warmup)
    ms = _time_ms(step, a.steps, a.warmup)
    flops = chunks * 2 * (2 * C * C * D + 2 * C * C * D + 2 * C * D * D + C * C * D + C * D * D)
    tf = 3 * flops / (ms * 1e-3) / 1e12
    dk = kern[dom]
    print(json.dumps({
        "metric": "Gated DeltaNet chunked scan fwd+bwd tokens/sec @1 GPU", "value": round(B * T / (ms * 1e-3), 1),
        "unit": "tokens/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16 in/out, f32 arithmetic",
        "data": "synthetic normals (l2-normalised keys)",
        "config": {"workload": f"chunked gated delta rule fwd+bwd B={B} T={T} H={H} Dk=Dv={D} chunk={C} "
                               "(configs/stage1.yml GDN shape)"},
        "fwd": {"ms": round(ms_f, 4), "tokens_s": round(B * T / (ms_f * 1e-3), 1),
                "TFLOP/s": round(flops / (ms_f * 1e-3) / 1e12, 2), "note": "inference forward (no residuals kept)"},
        "fwd_save": {"ms": round(ms_fs, 4), "saved_MB": round(saved.numel() / 1e6, 1),
                     "note": "training forward: also keeps the chunk products and the state entering every chunk"},
        "bwd": {"ms": round(ms_b, 4), "TFLOP/s": round(2 * flops / (ms_b * 1e-3) / 1e12, 2),
                "note": "from the kept residuals"},
        "recompute": {"bwd_ms": round(ms_br, 4), "fwd_bwd_ms": round(ms_r, 4),
                      "note": "backward recomputing the forward's chunk products and states (nothing kept)"},
        "kernels": kern,
        "roofline": {"kernel": dom, "bound": "hbm", "achieved": dk["GB/s"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": dk["hbm_frac"], "traffic": dk["traffic"], "launch_ms": dk["ms"],
                     "note": "the step's longest kernel against HBM: achieved = its algorithmic bytes (tiles read and "
                             "written once per chunk) / its average launch time; traffic = rocprofv3 FETCH_SIZE + "
                             "WRITE_SIZE bytes per launch (profiles/gdn_chunked_fwd_bwd.md)"},
        "matrix_view": {"achieved": round(tf, 2), "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(tf / PEAK_FP32_TFLOPS, 4),
                        "note": "the whole step's algorithmic f32 flops (counted once; the products run on the bf16 "
                                "matrix cores as hi/lo terms) over the fp32 matrix peak"}}), flush=True)


def gdn_kernel_bytes(C, D):
    """Algorithmic HBM bytes per (chunk, head, sequence) of each chunked gated delta rule kernel of the training step
    (read, written): every tile read or written once.  bf16 [C, D] tiles are 2 C D bytes, f32 [C, C] 4 C C, the f32
    state [D, D] 4 D D; per-token scalars (g, beta, gcum, dg, dbeta) 4 C or 2 C.
      gdn_chunk   reads q, k, v, g, beta; writes u, w, attn, gcum and the backward's S, A
      gdn_scan    reads q, k, w, u, attn, gcum; writes o and the state entering the chunk
      gdn_bscan   reads q, k, w, attn, gcum, do; writes dH entering the chunk
      gdn_bgrad   reads k, u, w, attn, gcum, do, h, dH; writes dqg, dkd (f32), du, dw (bf16), dP (f32), dgl
      gdn_bchunk  reads q, k, v, beta, attn, gcum, S, A, dqg, dkd, du, dw, dP, dgl; writes dq, dk, dv, dg, dbeta"""
    t16, m32, st, sc = 2 * C * D, 4 * C * C, 4 * D * D, 4 * C
    return {
        "gdn_chunk": (3 * t16 + sc + 2 * C, 2 * t16 + 3 * m32 + sc),
        "gdn_scan": (4 * t16 + m32 + sc, t16 + st),
        "gdn_bscan": (4 * t16 + m32 + sc, st),
        "gdn_bgrad": (4 * t16 + m32 + sc + 2 * st, 2 * 2 * t16 + 2 * t16 + m32 + 4),
        "gdn_bchunk": (3 * t16 + 2 * C + 3 * m32 + sc + 2 * 2 * t16 + 2 * t16 + m32 + 4, 3 * t16 + 2 * sc),
    }


def _time_ms(fn, steps, warmup):
    """Mean ms per call of fn, HIP events on torch's current stream (where the kernels are launched)."""
    import torch
    for _ in range(warmup):
        fn()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def permute_bench(a):
    """The drop-in permute kernels at the shapes of the reference's own microbench (colab/tpu_permute_bench.py:22-104:
    N = 8 x 4096 tokens, D = 1024, E = 128, k in {6, 12}): gather_rows, gather_reduce, gather_dot, sort_indices
    (argsort vs count, both the same counting-sort kernel here), and the dispatch -> identity expert -> combine block
    forward + backward.  GB/s use the reference's byte model, read + write of the gathered rows (line 63), per kernel:
    gather_rows 2 M D 2, gather_reduce M D 2 + N D 2 (bf16 out), gather_dot M D 2 + N D 2, and for the block the sum
    over its kernels of their byte models (dispatch 2 M D 2, combine M D 2 + N D 4, combine backward dy 2 M D 2 and
    dw M D 2 + N D 2, dispatch backward M D 2 + N D 2; index bytes included).  Beside every kernel, the reference
    column: the same call through the plain torch path (CFG["enabled"] = False) and the block with
    use_kernels=False, as the reference times its XLA path (colab/tpu_permute_bench.py:72-77, 96-104)."""
    import torch

    import moe_permute as mp

    dev = torch.device("cuda", 0)
    E, N, D = 128, 8 * 4096, 1024
    out = {}
    for k in (6, 12):
        M = N * k
        gen = torch.Generator(device=dev).manual_seed(0)
        x = torch.randn((N, D), device=dev, generator=gen).to(torch.bfloat16)
        sel = torch.argsort(-torch.randn((N, E), device=dev, generator=gen), dim=1, stable=True)[:, :k].to(torch.int32)
        flat = sel.reshape(-1).contiguous()
        w = torch.softmax(torch.randn((N, k), device=dev, generator=gen), dim=1)
        y = torch.randn((M, D), device=dev, generator=gen).to(torch.bfloat16)
        g = torch.randn((N, D), device=dev, generator=gen).to(torch.bfloat16)
        order, pos = mp.sort_indices(flat, E)
        idx = torch.div(order, k, rounding_mode="floor").to(torch.int32)
        pos2 = pos.reshape(N, k)
        res = {}

        def both(fn, steps, warmup):
            """(kernel ms, reference ms): the reference column is the same call with CFG["enabled"] = False, the
            plain torch path (the reference times its XLA path the same way, colab/tpu_permute_bench.py:72-77)."""
            tk = _time_ms(fn, steps, warmup)
            mp.CFG["enabled"] = False
            try:
                tr = _time_ms(fn, steps, warmup)
            finally:
                mp.CFG["enabled"] = True
            return tk, tr

        t, tr = both(lambda: mp.sort_indices(flat, E, "count"), a.steps, a.warmup)
        res["sort_indices"] = dict(ms=round(t, 4), GBs=round((4 * M + 8 * M) / (t * 1e-3) / 1e9, 1),
                                   ref_ms=round(tr, 4), ref_note="torch.argsort(flat) and argsort(argsort(flat))")
        for name, fn, nbytes in (
                ("gather_rows", lambda: mp.gather_rows(x, idx), 2 * M * D * 2 + 4 * M),
                ("gather_reduce", lambda: mp.gather_reduce(y, pos2, w), M * D * 2 + N * D * 2 + 8 * M),
                ("gather_dot", lambda: mp.gather_dot(y, pos2, g), M * D * 2 + N * D * 2 + 8 * M)):
            t, tr = both(fn, a.steps, a.warmup)
            res[name] = dict(ms=round(t, 4), GBs=round(nbytes / (t * 1e-3) / 1e9, 1), ref_ms=round(tr, 4),
                             ref_GBs=round(nbytes / (tr * 1e-3) / 1e9, 1), speedup=round(tr / t, 2))
        mp.CFG["num_experts"] = E
        try:
            xg = x.clone().requires_grad_(True)
            wg = w.clone().requires_grad_(True)
            gf = g.float()

            def block(use):
                xg.grad = None
                wg.grad = None
                o = mp.moe_block(xg, flat, wg, lambda r: r, use_kernels=use)
                (o * gf).sum().backward()

            bs, bw = max(5, a.steps // 4), max(2, a.warmup // 4)
            t = _time_ms(lambda: block(True), bs, bw)
            tr = _time_ms(lambda: block(False), bs, bw)
        finally:
            mp.CFG["num_experts"] = None
        model = (2 * M * D * 2 + 4 * M) + (M * D * 2 + N * D * 4 + 8 * N * k) + (2 * M * D * 2 + 8 * M) \
            + (M * D * 2 + N * D * 2 + 4 * N * k) + (M * D * 2 + N * D * 2 + 4 * N * k)
        res["block_fwd_bwd"] = dict(ms=round(t, 4), GBs=round(model / (t * 1e-3) / 1e9, 1), ref_ms=round(tr, 4),
                                    speedup=round(tr / t, 2),
                                    note="sort + dispatch + combine fwd, fused combine bwd + dispatch bwd, torch glue "
                                         "(the loss reduction) included; the reference column is "
                                         "moe_block(use_kernels=False): ref_dispatch / ref_combine under torch autograd "
                                         "(colab/tpu_permute_bench.py:96-104)")
        out[f"k={k}"] = res
    k6 = out["k=6"]["gather_rows"]["GBs"]
    print(json.dumps({
        "metric": "MoE permute kernels GB/s @1 GPU (reference microbench shapes)", "value": k6, "unit": "GB/s",
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": out["k=6"]["gather_rows"]["ms"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16 rows, f32 reductions",
        "data": "synthetic normals, top-k of random logits",
        "config": {"workload": f"colab/tpu_permute_bench.py shapes: N={N} D={D} E={E} k in (6, 12)"},
        "kernels": out,
        "roofline": {"kernel": "gather_rows (k=6)", "bound": "hbm", "achieved": k6, "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(k6 / PEAK_HBM_GBS, 4), "traffic": None}}), flush=True)


def ragged_bench(a):
    """lsurge_ragged_dot (forward) and lsurge_ragged_dot_bwd (dlhs + drhs) at the MoE layer's per-weight shapes, the
    pattern of the reference's GEMM ceiling bench (modal/gemm_bench.py:25-35: up, down and dW per weight): C2's
    routing (M = 98304 rows in 64 groups from the layer's own top-6 of seeded logits), wi_0 / wi_1 [1024 -> 512] and
    wo [512 -> 1024]; plus the reference's 8192^3 ceiling (one group) and torch.matmul (hipBLASLt) on the same dense
    shapes for context.  TF/s count useful rows only."""
    import torch

    import numpy as np

    import _lib as L

    dev = torch.device("cuda", 0)
    lib = L.lib()
    st = L.stream(dev)
    c = CONFIGS["C2"]
    rng = np.random.default_rng(0)
    # the top-k of seeded logits, ties to the lower expert index (a stable sort of the negated logits)
    sel = np.argsort(-rng.standard_normal((c["T"], c["E"])).astype("float32"), axis=1, kind="stable")[:, :c["k"]]
    gs_np = np.bincount(sel.reshape(-1), minlength=c["E"]).astype("int32")
    M, E = int(gs_np.sum()), c["E"]
    gs = torch.from_numpy(gs_np).to(dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    res = {}
    for name, K, Nn in (("up (wi_0 / wi_1) 1024->512", 1024, 512), ("down (wo) 512->1024", 512, 1024)):
        lhs = torch.randn((M, K), device=dev, generator=gen).to(torch.bfloat16)
        rhs = (torch.randn((E, K, Nn), device=dev, generator=gen) * 0.02).to(torch.bfloat16)
        g = torch.randn((M, Nn), device=dev, generator=gen).to(torch.bfloat16)
        out = torch.empty((M, Nn), dtype=torch.bfloat16, device=dev)
        dl = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
        dr = torch.empty((E, K, Nn), dtype=torch.float32, device=dev)
        ws = L.workspace(lib.lsurge_ragged_dot_bwd_workspace_bytes(M, K, Nn, E), dev)
        fl = 2 * M * K * Nn

        def fwd():
            L.check(lib.lsurge_ragged_dot(L.ptr(lhs), L.ptr(rhs), L.ptr(gs), M, K, Nn, E, L.BF16, L.ptr(out), L.BF16,
                                          L.ptr(ws), ws.numel(), st), "ragged_dot")

        def bwd():
            L.check(lib.lsurge_ragged_dot_bwd(L.ptr(lhs), L.ptr(rhs), L.ptr(gs), L.ptr(g), M, K, Nn, E, L.BF16, L.ptr(dl),
                                              L.ptr(dr), L.ptr(ws), ws.numel(), st), "ragged_dot_bwd")

        tf, tb = _time_ms(fwd, a.steps, a.warmup), _time_ms(bwd, a.steps, a.warmup)
        dense = torch.randn((M, K), device=dev, generator=gen).to(torch.bfloat16)
        wd = rhs[0].contiguous()
        th = _time_ms(lambda: torch.matmul(dense, wd), a.steps, a.warmup)
        res[name] = dict(fwd_ms=round(tf, 4), fwd_TFs=round(fl / (tf * 1e-3) / 1e12, 1), bwd_ms=round(tb, 4),
                         bwd_TFs=round(2 * fl / (tb * 1e-3) / 1e12, 1),
                         hipblaslt_dense_same_shape_TFs=round(fl / (th * 1e-3) / 1e12, 1))
    # f32 operands at the up shape: three bf16 terms per value, six term products (a GEMM six times as deep) plus the
    # split kernels; TF/s count the f32 product's 2 M K N, against the fp32 matrix peak
    K, Nn = 1024, 512
    lhs = torch.randn((M, K), device=dev, generator=gen)
    rhs = torch.randn((E, K, Nn), device=dev, generator=gen) * 0.02
    g = torch.randn((M, Nn), device=dev, generator=gen)
    out = torch.empty((M, Nn), dtype=torch.float32, device=dev)
    dl = torch.empty((M, K), dtype=torch.float32, device=dev)
    dr = torch.empty((E, K, Nn), dtype=torch.float32, device=dev)
    ws = L.workspace(max(lib.lsurge_ragged_dot_f32_workspace_bytes(M, K, Nn, E),
                         lib.lsurge_ragged_dot_bwd_f32_workspace_bytes(M, K, Nn, E)), dev)
    fl = 2 * M * K * Nn
    tf = _time_ms(lambda: L.check(lib.lsurge_ragged_dot(L.ptr(lhs), L.ptr(rhs), L.ptr(gs), M, K, Nn, E, L.F32,
                                                        L.ptr(out), L.F32, L.ptr(ws), ws.numel(), st), "rd f32"),
                  a.steps, a.warmup)
    tb = _time_ms(lambda: L.check(lib.lsurge_ragged_dot_bwd(L.ptr(lhs), L.ptr(rhs), L.ptr(gs), L.ptr(g), M, K, Nn, E,
                                                            L.F32, L.ptr(dl), L.ptr(dr), L.ptr(ws), ws.numel(), st),
                                  "rd f32 bwd"), a.steps, a.warmup)
    res["up 1024->512, f32 operands (3 bf16 terms, 6 products)"] = dict(
        fwd_ms=round(tf, 4), fwd_TFs=round(fl / (tf * 1e-3) / 1e12, 1), bwd_ms=round(tb, 4),
        bwd_TFs=round(2 * fl / (tb * 1e-3) / 1e12, 1), fp32_matrix_peak_TFs=PEAK_FP32_TFLOPS)
    del lhs, rhs, g, out, dl, dr, ws
    big = torch.randn((8192, 8192), device=dev, generator=gen).to(torch.bfloat16)
    out = torch.empty_like(big)
    one = torch.tensor([8192], dtype=torch.int32, device=dev)
    ws = L.workspace(lib.lsurge_ragged_dot_workspace_bytes(8192, 1), dev)
    bigt = big.t().contiguous()
    t8 = _time_ms(lambda: L.check(lib.lsurge_ragged_dot(L.ptr(big), L.ptr(bigt), L.ptr(one), 8192, 8192, 8192, 1,
                                                         L.BF16, L.ptr(out), L.BF16, L.ptr(ws), ws.numel(), st), "rd"),
                  max(3, a.steps // 4), 2)
    t8h = _time_ms(lambda: torch.matmul(big, big), max(3, a.steps // 4), 2)
    res["reference 8192^3 (one group)"] = dict(ms=round(t8, 4), TFs=round(2 * 8192 ** 3 / (t8 * 1e-3) / 1e12, 1),
                                               hipblaslt_TFs=round(2 * 8192 ** 3 / (t8h * 1e-3) / 1e12, 1))
    up = res["up (wi_0 / wi_1) 1024->512"]["fwd_TFs"]
    print(json.dumps({
        "metric": "ragged_dot (padded_gmm drop-in) TFLOP/s @1 GPU, layer per-weight shapes", "value": up,
        "unit": "TFLOP/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": res["up (wi_0 / wi_1) 1024->512"]["fwd_ms"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 (f32 accumulation)", "data": "synthetic normals; C2 group sizes",
        "config": {"workload": f"ragged_dot M={M} E={E} (C2 routing), per-weight shapes of modal/gemm_bench.py"},
        "kernels": res,
        "roofline": {"kernel": "ragged_dot up fwd", "bound": "mfma", "achieved": up, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(up / PEAK_BF16_TFLOPS, 4), "traffic": None}}), flush=True)

def mfma_sustained(iters=2000, reps=3):
    """The matrix cores' sustained bf16 rate on register-resident operands (lsurge_mfma_rate_probe, no memory traffic):
    pseudo-random values and zeros, TFLOP/s from HIP events on the probe's stream, best of `reps` after a warm-up
    launch.  Random operands draw more power than zeros, and the chip's power limit holds them below the datasheet
    peak: the rate a GEMM on real data can approach."""
    import torch
    import _lib as L
    dev = torch.device("cuda", torch.cuda.current_device())
    out = torch.empty(L.lib().lsurge_mfma_rate_probe_out_floats(), dtype=torch.float32, device=dev)
    flops = iters * float(2 ** 33)
    rates = {}
    for zero in (0, 1):
        L.check(L.lib().lsurge_mfma_rate_probe(zero, iters, L.ptr(out), L.stream(dev)), "mfma_rate_probe")
        best = 0.0
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            L.check(L.lib().lsurge_mfma_rate_probe(zero, iters, L.ptr(out), L.stream(dev)), "mfma_rate_probe")
            e1.record()
            e1.synchronize()
            best = max(best, flops / (e0.elapsed_time(e1) * 1e-3) / 1e12)
        rates[zero] = best
    return {"random_bf16": round(rates[0], 1), "zero_operands": round(rates[1], 1), "unit": "TFLOP/s",
            "kernel": "mfma_rate_kernel (v_mfma_f32_32x32x16_bf16, operands in registers)"}


def layer_measure(a, c, steps, warmup):
    """Time `steps` fwd(+bwd) layer steps of config c after `warmup` (helper streams per a.concurrency), with a
    profiled one-stream pass first that finds the dominant kernel; that kernel is bracketed by HIP events on its
    launch stream during the timed steps.  Returns the step time, tokens/s, the per-kernel table and the roofline
    figures of the dominant kernel."""
    import torch

    import _lib
    from moe_layer import MoELayer, MoEShape

    dev = torch.device("cuda", 0)
    lib = _lib.lib()
    lib.lsurge_set_concurrency(0)
    p, dy = make_params(c, dev)
    layer = MoELayer(MoEShape(c["T"], c["d"], c["E"], c["k"], c["f"], c["fs"]), dev)
    grads = layer.alloc_grads() if c["bwd"] else None

    def step():
        if a.fp8:
            layer.quantize_weights_fp8(p)
            layer.forward_fp8(p)
            if c["bwd"]:
                layer.backward_fp8(p, dy, grads)
            return
        layer.forward(p)
        if c["bwd"]:
            layer.backward(p, dy, grads)

    for _ in range(2):  # first-call work (code objects, helper events) before the profiled pass
        step()
    torch.cuda.synchronize()

    # profiled pass (one stream, so every kernel's time is its own): every kernel bracketed, to find the
    # dominant one and fill the per-kernel table
    lib.lsurge_prof_reset()
    lib.lsurge_prof_enable(-1)
    nprof = 3
    for _ in range(nprof):
        step()
    torch.cuda.synchronize()
    lib.lsurge_prof_collect()
    lib.lsurge_prof_enable(0)
    table = prof_table(lib, nprof)
    work = kernel_work(c, a.fp8)
    dom = max((n for n in table if n in work), key=lambda n: table[n][2])
    names = [lib.lsurge_prof_kernel_name(i).decode() for i in range(lib.lsurge_prof_kernel_count())]

    # timed region: K steps, only the dominant kernel bracketed by events on its launch stream
    # the W warm-up steps run in the timed region's mode (helper streams): the step time settles only after ~20
    # back-to-back steps (measured: 2 steps leave the timed mean 3% high)
    lib.lsurge_set_concurrency(a.concurrency)
    for _ in range(warmup):
        step()
    lib.lsurge_prof_reset()
    lib.lsurge_prof_enable(1 << names.index(dom))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    lib.lsurge_prof_collect()
    lib.lsurge_prof_enable(0)
    timed = prof_table(lib, steps)
    dom_ms = timed[dom][0]
    bound, amount = work[dom]
    peak_mfma = PEAK_FP8_TFLOPS if a.fp8 else PEAK_BF16_TFLOPS
    if bound == "mfma":
        achieved, peak, unit = amount / (dom_ms * 1e-3) / 1e12, peak_mfma, "TFLOP/s"
    else:
        achieved, peak, unit = amount / (dom_ms * 1e-3) / 1e9, PEAK_HBM_GBS, "GB/s"
    ms = el / steps * 1e3
    cached_ms = None
    if a.fp8:  # the same step on weights quantised once
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            layer.forward_fp8(p)
            if c["bwd"]:
                layer.backward_fp8(p, dy, grads)
        torch.cuda.synchronize()
        cached_ms = (time.perf_counter() - t0) / steps * 1e3
    serial_ms = sum(v[2] for v in table.values())
    kern = {n: dict(ms=round(v[0], 4), share=round(v[2] / serial_ms, 4)) for n, v in sorted(table.items(),
                                                                                          key=lambda kv: -kv[1][2])}
    for n, v in kern.items():
        if n in work:
            b, amt = work[n]
            v["achieved"] = round(amt / (v["ms"] * 1e-3) / (1e12 if b == "mfma" else 1e9), 1)
            v["unit"] = "TFLOP/s" if b == "mfma" else "GB/s"
    lib.lsurge_set_concurrency(0)
    del layer, p, dy, grads
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return dict(ms=ms, tokens_s=c["T"] * steps / el, dom=dom, bound=bound, achieved=achieved, peak=peak, unit=unit,
                dom_ms=dom_ms, kern=kern, cached_ms=cached_ms, peak_mfma=peak_mfma)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="C2", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="C2 run: skip the C1, C3, C4, C5 lines appended to the JSON (configs key)")
    ap.add_argument("--other-steps", type=int, default=10, help="timed (and warm-up) steps of each other config")
    ap.add_argument("--fp8", action="store_true", help="expert GEMMs in FP8 (current scaling: E4M3 forward, E5M2 "
                    "gradients)")
    ap.add_argument("--fwd-only", action="store_true", help="time the forward alone")
    ap.add_argument("--op", choices=["moe", "conv", "gdn", "permute", "ragged_dot"], default="moe",
                    help="conv: the Gated DeltaNet block's causal depthwise Conv1D (modal/fast_conv.py) at the "
                         "reference config's shape, forward + backward GB/s; gdn: its chunked gated delta rule "
                         "(modal/gdn_fast.py), forward + backward tokens/s; permute: the moe_permute kernels at the shapes of "
                         "colab/tpu_permute_bench.py; ragged_dot: the padded_gmm drop-in at the layer's per-weight "
                         "shapes (modal/gemm_bench.py)")
    ap.add_argument("--kernels", action="store_true", help="also print the per-kernel table to stderr")
    ap.add_argument("--gemm-variant", type=int, default=1, choices=[0, 1],
                    help="grouped-GEMM kernels: 1 the persistent 256 x 256 kernel (default), 0 the classic 128 x 256 "
                         "and ping-pong kernels (lsurge_set_gemm_variant; bitwise identical results)")
    ap.add_argument("--concurrency", type=int, default=1,
                    help="timed region: 1 runs the layer's independent chains on helper streams "
                         "(lsurge_set_concurrency), 0 everything on one stream")
    ap.add_argument("--profile-summary", metavar="DIR", help="print the markdown summary of a rocprofv3 "
                    "--kernel-trace output directory of this bench (with --pmc-fetch/--pmc-write and "
                    "--copy-fetch/--copy-write counter directories for traffic) and exit")
    ap.add_argument("--stats-summary", metavar="DIR", help="print the kernel table of a rocprofv3 --stats run and exit")
    ap.add_argument("--kernel-traffic", action="store_true", help="print per-kernel HBM bytes per launch from the "
                    "--pmc-fetch / --pmc-write counter runs (calibrated by --copy-fetch / --copy-write) and exit")
    ap.add_argument("--pmc-fetch", metavar="DIR")
    ap.add_argument("--pmc-write", metavar="DIR")
    ap.add_argument("--copy-fetch", metavar="DIR")
    ap.add_argument("--copy-write", metavar="DIR")
    ap.add_argument("--copy-probe-mib", type=int, default=1024, help="size of the --copy-probe run being calibrated on")
    ap.add_argument("--pmc-extra", metavar="DIR", action="append", default=[],
                    help="with --profile-summary: rocprofv3 --pmc output directories of further counter passes "
                         "(clock, MFMA utilisation, LDS and TA/TD activity per role)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB three times (calibrates rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE against a known byte count) and exit")
    a = ap.parse_args()
    if a.gpus != 1:
        print("bench.py: this build measures one GPU only (the MoE layer at one GPU's share); "
              f"--gpus {a.gpus} is not supported", file=sys.stderr)
        sys.exit(2)

    if a.stats_summary:
        stats_summary(a.stats_summary)
        return
    if a.kernel_traffic:
        kernel_traffic(a)
        return
    if a.profile_summary:
        profile_summary(a)
        return

    import torch

    if not a.copy_probe:
        import _lib as _vlib
        _vlib.check(_vlib.lib().lsurge_set_gemm_variant(a.gemm_variant), "set_gemm_variant")

    if a.copy_probe:
        n = a.copy_probe << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_read": n, "copy_probe_bytes_written": n, "launches": 3}), flush=True)
        return

    if a.op == "conv":
        conv_bench(a)
        return
    if a.op == "gdn":
        gdn_bench(a)
        return
    if a.op == "permute":
        permute_bench(a)
        return
    if a.op == "ragged_dot":
        ragged_bench(a)
        return

    c = CONFIGS[a.config]
    if a.fwd_only:
        c = dict(c, bwd=False)
    m = layer_measure(a, c, a.steps, a.warmup)
    ms, tokens_s, dom, bound, achieved, peak, unit, dom_ms, kern, cached_ms, peak_mfma = (
        m["ms"], m["tokens_s"], m["dom"], m["bound"], m["achieved"], m["peak"], m["unit"], m["dom_ms"], m["kern"],
        m["cached_ms"], m["peak_mfma"])
    if a.kernels:
        for n, v in kern.items():
            print(f"  {n:20s} {v}", file=sys.stderr)
    sus = mfma_sustained()
    if bound == "mfma":
        sus["roofline_frac_of_sustained"] = round(achieved / sus["random_bf16"], 4)

    res = {
        "metric": (f"MoE-layer {'fwd+bwd' if c['bwd'] else 'fwd'} tokens/sec @1 GPU, FP8 expert GEMMs" if a.fp8 else
                   "MoE-layer fwd+bwd tokens/sec @1 GPU; GEMM MFMA util %, permute HBM GB/s"),
        "value": round(tokens_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("fp8 expert GEMMs: e4m3 activations and weights, e5m2 gradients (bf16 router, combine, saved "
                  "activations)" if a.fp8 else "bf16"),
        "data": "synthetic (torch seeded normals: x~N(0,1), weights~N(0,0.02), dy~N(0,1), bf16), resident in HBM",
        "config": {"workload": f"{a.config}: MoE layer {'fwd+bwd' if c['bwd'] else 'fwd'}{' fp8' if a.fp8 else ''} T={c['T']} d={c['d']} "
                               f"E={c['E']}x{c['f']} top-{c['k']} shared={c['fs']}" + (" zipf-bias" if c["zipf"] else ""),
                   "T": c["T"], "d_model": c["d"], "experts": c["E"], "top_k": c["k"], "expert_ffn": c["f"],
                   "shared_ffn": c["fs"], "block_rows": 128, "parallelism": "single GPU",
                   "concurrent_streams": bool(a.concurrency), "gemm_variant": a.gemm_variant},
        "layer_tflops": round(layer_flops(c) / (ms * 1e-3) / 1e12, 1),
        "mfu": round(layer_flops(c) / (ms * 1e-3) / 1e12 / peak_mfma, 4),
        "roofline": {"kernel": dom, "bound": bound, "achieved": round(achieved, 1), "peak": peak, "unit": unit,
                     "frac": round(achieved / peak, 4), "traffic": measured_traffic(a.config, dom, a.fp8, c["bwd"]),
                     "launch_ms": round(dom_ms, 4)},
        "kernels": kern,
        "mfma_sustained": sus,
        **({"ms_per_step_cached_weights": round(cached_ms, 4),
            "tokens_s_cached_weights": round(c["T"] / (cached_ms * 1e-3), 1)} if a.fp8 else {}),
        "kernels_note": "per-kernel ms from a profiled pass on one stream (share of that pass's kernel time); "
                        "the timed region runs with concurrent_streams",
    }
    if a.config == "C2" and c["bwd"] and not a.fp8 and not a.no_other_configs:
        # every other BASELINE config on the same line: a few timed steps each, with its dominant kernel's roofline
        # (no CPU baseline for these)
        res["configs"] = {}
        for name in ("C1", "C3", "C4", "C5"):
            cc = CONFIGS[name]
            mm = layer_measure(a, cc, a.other_steps, a.other_steps)
            res["configs"][name] = {
                "workload": f"{name}: MoE layer {'fwd+bwd' if cc['bwd'] else 'fwd'} T={cc['T']} d={cc['d']} "
                            f"E={cc['E']}x{cc['f']} top-{cc['k']} shared={cc['fs']}" + (" zipf-bias" if cc["zipf"] else ""),
                "steps": a.other_steps, "warmup": a.other_steps, "ms_per_step": round(mm["ms"], 4),
                "tokens_s": round(mm["tokens_s"], 1),
                "layer_tflops": round(layer_flops(cc) / (mm["ms"] * 1e-3) / 1e12, 1),
                "mfu": round(layer_flops(cc) / (mm["ms"] * 1e-3) / 1e12 / mm["peak_mfma"], 4),
                "roofline": {"kernel": mm["dom"], "bound": mm["bound"], "achieved": round(mm["achieved"], 1),
                             "peak": mm["peak"], "unit": mm["unit"], "frac": round(mm["achieved"] / mm["peak"], 4),
                             "launch_ms": round(mm["dom_ms"], 4)},
                "kernels": {n: v for n, v in list(mm["kern"].items())[:8]},
            }
    if not a.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(c)
        if a.config == "C2" and c["bwd"]:  # BASELINE.md's pair: C1 forward beside C2 forward + backward
            res["cpu_baseline_c1_fwd"] = cpu_baseline(CONFIGS["C1"], target_s=5.0)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
