"""Benchmark: Pairformer layers/s at N=512 on one MI355X (BASELINE.json metric).

A step is one full Boltz-2 PairformerLayer (triangle multiplication out+in,
triangle attention start+end, pair transition, single attention with pair bias,
single transition) applied in place to device-resident z [1,512,512,128] fp32 and
s [1,512,384] fp32, masks all ones, random-init weights from seed 0 (the
config-0 layer architecture), fp16 MFMA operands with fp32 accumulation (the bf16-operand
build of the same kernels is timed beside it).

Besides the JSON line's ``value`` (layers/s), it reports per-op times and
TFLOP/s, the roofline of the dominant kernel (the triangle-attention core, its launches
timed inside the layer loop with HIP events on the stream it is launched on, with its VALU
roof and the chip's sustained MFMA rate beside the nameplate peak), the same for the trimul
contraction, and the CPU oracle timed on this host's cores.

The config-3 trunk (64 layers at N=768, recycling_steps=3 -> 4 passes, device
resident) and the contraction alone at N=768 are reported under ``stack``.

``--probe-traffic`` runs only the attention core and the contraction (5 launches each
at N=512) and a plain copy kernel of known size, for ``rocprofv3 --pmc FETCH_SIZE`` /
``WRITE_SIZE`` runs; the calibrated per-launch traffic is read back from
``profiles/kernel_traffic_n512.json`` when that file exists.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--n 512] [--no-cpu-baseline]
                       [--no-stack] [--probe-traffic] [--probe-contract]
"""
from __future__ import annotations

import argparse
from typing import Optional
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

MFMA_BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 / fp16 (AMD published)
HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "kernel_traffic_n512.json")
COPY_BYTES = 256 << 20            # the calibration copy kernel reads and writes this many bytes


def flops_layer(N: int, c: int = 128, hd: int = 128, H: int = 4, c_s: int = 384) -> dict:
    """Algorithmic FLOP per op for one layer (matmul-like terms only)."""
    tm_contract = 2 * N ** 3 * c
    tm_proj = 12 * N ** 2 * c * c
    ta_core = 4 * N ** 3 * hd
    ta_proj = 2 * N ** 2 * c * (4 * hd + H) + 2 * N ** 2 * hd * c
    tr = 24 * N ** 2 * c * c
    s_track = (2 * N ** 2 * c * 16 + 2 * N * c_s * c_s * 5 + 4 * N ** 2 * c_s + 2 * N * c_s * 4 * c_s * 3)
    return {"trimul": tm_contract + tm_proj, "trimul_contract": tm_contract, "triatt": ta_core + ta_proj,
            "triatt_core": ta_core, "transition_z": tr, "s_track": s_track,
            "layer": 2 * (tm_contract + tm_proj) + 2 * (ta_core + ta_proj) + tr + s_track}


def cpu_baseline(N: int, seed: int, reps: int = 3) -> dict:
    """Time the fp32 CPU oracle for one layer at this N on the host cores (median of reps)."""
    import torch
    from oracle import pairformer_ref as ref
    from tt_boltz_amd import synthetic
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    w = synthetic.stack_weights(1, seed)
    s, z, mask, pm = synthetic.pair_inputs(N, seed)
    lw = ref.sub(w, "layers.0")
    chunk = ref.chunk_size_for(N)
    with torch.no_grad():
        ref.pairformer_layer(s, z, mask, pm, lw, chunk)          # warm-up
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            ref.pairformer_layer(s, z, mask, pm, lw, chunk)
            ts.append(time.perf_counter() - t0)
    ts.sort()
    sec = ts[len(ts) // 2]
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": 1.0 / sec, "unit": "layers/s", "cores": cores, "kind": "port",
            "sample": f"1 PairformerLayer at N={N}, fp32 CPU oracle (oracle/pairformer_ref.py), torch "
                      f"{torch.__version__}, {cores} threads, median of {reps} after 1 warm-up; "
                      f"{sec:.2f} s/layer; cpu={cpu}"}


def cpu_configs(reps: int = 3) -> dict:
    """The CPU oracle against this build's GPU path on the BASELINE configs, per op where the
    config is per op: config 0 (one layer at N = 128, in full), configs 1 / 2 (each triangle
    multiplication / attention at N = 512 with the 51-token padded tail), and a bounded sample of
    config 4 (the block-fp8 emulator's triangle multiplication and pair transition at N = 512
    against the fast-mode kernels at the same N; the emulator runs once, its N = 1024 case would
    take minutes).  CPU: fp32 oracle, all host threads, median of `reps` after one warm-up (one
    run for the emulator).  GPU: HIP events, device-resident inputs, same weights and inputs."""
    import torch
    from oracle import pairformer_ref as ref
    from tt_boltz_amd import ops, pairformer, synthetic
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    dev = pairformer.get_device()
    stream = torch.cuda.current_stream()

    def cpu_s(fn, n):
        with torch.no_grad():
            if n > 1:
                fn()
            ts = []
            for _ in range(n):
                t0 = time.perf_counter()
                fn()
                ts.append(time.perf_counter() - t0)
        ts.sort()
        return ts[len(ts) // 2]

    def entry(c_s, g_ms):
        return {"cpu_s": round(c_s, 4), "gpu_ms": round(g_ms, 4), "gpu_speedup": round(c_s * 1e3 / g_ms, 1)}

    res = {"cores": cores, "torch": torch.__version__}
    # config 0: one PairformerLayer at N = 128
    cfg = synthetic.CONFIGS[0]
    N = cfg["N"]
    w = synthetic.stack_weights(1, cfg["seed"])
    s, z, mask, pm = synthetic.pair_inputs(N, cfg["seed"])
    lw = ref.sub(w, "layers.0")
    c = cpu_s(lambda: ref.pairformer_layer(s, z, mask, pm, lw, ref.chunk_size_for(N)), reps)
    pf = pairformer.Pairformer(1, 32, 4, 24, 16, True, w)
    ws = ops.workspace(pf.workspace_bytes(1, N), dev)
    zd, sd = z.to(dev).contiguous(), s.to(dev).contiguous()
    md, pmd = mask.to(dev).contiguous(), pm.to(dev).contiguous()
    res["config0_layer_n128"] = entry(c, time_events(lambda: pf.blocks[0](sd, zd, pmd, md, ws), 20, stream))
    del pf, ws
    # configs 1 and 2: the four triangle ops at N = 512, padded tail
    for k, ops_ in ((1, (("trimul_out", "tri_mul_out", "outgoing"), ("trimul_in", "tri_mul_in", "incoming"))),
                    (2, (("triatt_start", "tri_att_start", True), ("triatt_end", "tri_att_end", False)))):
        cfg = synthetic.CONFIGS[k]
        N = cfg["N"]
        w = synthetic.stack_weights(1, cfg["seed"])
        _, z, _, pm = synthetic.pair_inputs(N, cfg["seed"], pad_tail=cfg["pad_tail"], with_s=False)
        lw = ref.sub(w, "layers.0")
        layer = pairformer.Pairformer(1, 32, 4, 24, 16, True, w).blocks[0]
        ws = ops.workspace(layer.workspace_bytes(1, N), dev)
        zd, pmd = z.to(dev).contiguous(), pm.to(dev).contiguous()
        out = torch.empty_like(zd)
        for name, prefix, arg in ops_:
            if k == 1:
                c = cpu_s(lambda: ref.triangle_multiplication(z, pm, ref.sub(lw, prefix), arg), reps)
                mod = layer.triangle_multiplication_start if arg == "outgoing" else layer.triangle_multiplication_end
            else:
                c = cpu_s(lambda: ref.triangle_attention(z, pm, ref.sub(lw, prefix), arg,
                                                         ref.chunk_size_for(N)), reps)
                mod = layer.triangle_attention_start if arg else layer.triangle_attention_end
            res[f"config{k}_{name}_n{N}"] = entry(c, time_events(lambda: mod(zd, pmd, out=out, ws=ws), 10, stream))
        del layer, ws
    # config 4 sample: the block-fp8 emulator at N = 512
    cfg = synthetic.CONFIGS[4]
    N = 512
    w = synthetic.stack_weights(1, cfg["seed"])
    _, z, _, pm = synthetic.pair_inputs(N, cfg["seed"], with_s=False)
    lw = ref.sub(w, "layers.0")
    pairformer.set_fast_mode(True)
    try:
        layer = pairformer.Pairformer(1, 32, 4, 24, 16, True, w).blocks[0]
    finally:
        pairformer.set_fast_mode(False)
    ws = ops.workspace(layer.workspace_bytes(1, N), dev)
    zd, pmd = z.to(dev).contiguous(), pm.to(dev).contiguous()
    out = torch.empty_like(zd)
    c = cpu_s(lambda: ref.triangle_multiplication_mx8(z, pm, ref.sub(lw, "tri_mul_out"), "outgoing"), 1)
    res["config4_sample_trimul_out_mx8_n512"] = entry(
        c, time_events(lambda: layer.triangle_multiplication_start(zd, pmd, out=out, ws=ws), 10, stream))
    c = cpu_s(lambda: ref.transition_mx8(z, ref.sub(lw, "transition_z")), 1)
    tr_ws = ws[:layer.transition_workspace_bytes(1, N)] if layer.transition_workspace_bytes(1, N) else None
    res["config4_sample_transition_mx8_n512"] = entry(
        c, time_events(lambda: layer.transition_z(zd, out=out, ws=tr_ws), 10, stream))
    del layer, ws
    res["note"] = ("CPU: fp32 oracle (oracle/pairformer_ref.py; config 4: the block-fp8 emulator, "
                   "oracle/fp8_emu.py, one run), median of the runs after one warm-up; GPU: this build "
                   "on device-resident inputs; config 3 is stack.cpu_extrapolated")
    return res


def probe_traffic(N: int) -> int:
    """The roofline kernels alone on their real operands -- the triangle-attention core and
    the trimul contraction, 5 launches each -- and a plain copy kernel of COPY_BYTES read +
    COPY_BYTES written, for PMC runs (FETCH_SIZE / WRITE_SIZE)."""
    import torch
    from tt_boltz_amd import ops, pairformer, synthetic
    dev = torch.device("cuda", 0)
    pf = pairformer.Pairformer(1, 32, 4, 24, 16, True, synthetic.stack_weights(1, 0))
    layer = pf.blocks[0]
    _, z_cpu, _, _ = synthetic.pair_inputs(N, 0, with_s=False)
    z = z_cpu.to(dev).contiguous()
    ws = ops.workspace(pf.workspace_bytes(1, N), dev)
    layer.triangle_attention_start(z, None, out=torch.empty_like(z), ws=ws)
    torch.cuda.synchronize()
    for _ in range(5):
        ops.launch_triatt_attend(ws, 1, N, 0, layer.variant)
    g = torch.Generator(device=dev).manual_seed(0)
    A = torch.randn((128, N, N), device=dev, generator=g).half()
    Bm = torch.randn((128, N, N), device=dev, generator=g).half()
    X = torch.empty((128, N, N), dtype=torch.float16, device=dev)
    src = torch.randn(COPY_BYTES // 4, device=dev, generator=g)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        ops.launch_trimul_contract(A, Bm, X)
    for _ in range(3):
        torch.mul(src, 2.0, out=dst)     # vectorized elementwise kernel: reads and writes COPY_BYTES
    torch.cuda.synchronize()
    # three full layers (serial schedule, single track included) for the per-kernel summary
    s = synthetic.pair_inputs(N, 0)[0].to(dev).contiguous()
    for _ in range(3):
        layer(s, z, None, None, ws)
    torch.cuda.synchronize()
    print(json.dumps({"probe": "traffic", "N": N, "attn_launches": 5, "contract_launches": 5, "copy_launches": 3,
                      "copy_bytes": COPY_BYTES, "layer_launches": 3}), flush=True)
    return 0


CONTRACT_SIZES = (512, 768, 1024)


def probe_contract() -> int:
    """The 16-bit trimul contraction and the vendor library on the same [128, N, N] fp16 planes at
    N = 512, 768, 1024, 5 launches each, for rocprofv3 runs: X = A B^T through
    pf_trimul_contract (fp16 output), then torch.bmm(A, B^T) (hipBLASLt; B^T materialized once,
    so the library sees contiguous operands)."""
    import torch
    from tt_boltz_amd import ops
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    for N in CONTRACT_SIZES:
        A = torch.randn((128, N, N), device=dev, generator=g).half()
        Bm = torch.randn((128, N, N), device=dev, generator=g).half()
        Bt = Bm.transpose(1, 2).contiguous()
        X = torch.empty((128, N, N), dtype=torch.float16, device=dev)
        torch.cuda.synchronize()
        for _ in range(5):
            ops.launch_trimul_contract(A, Bm, X)
        torch.cuda.synchronize()
        for _ in range(5):
            torch.bmm(A, Bt, out=X)
        torch.cuda.synchronize()
        del A, Bm, Bt, X
        torch.cuda.empty_cache()
    print(json.dumps({"probe": "contract", "sizes": CONTRACT_SIZES, "launches": 5}), flush=True)
    return 0


CONTRACT_PMC_PASSES = ("SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_INST_ANY SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT "
                       "SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_MFMA GRBM_GUI_ACTIVE",
                       "SQ_WAIT_ANY SQ_INSTS_VALU SQ_INSTS_SALU SQ_ACTIVE_INST_LDS SQ_INSTS_VMEM_RD SQ_WAVE_CYCLES "
                       "GRBM_GUI_ACTIVE FETCH_SIZE")


def summarize_contract(kt_dir: str, pmc_dirs) -> None:
    """profiles/contract_vs_hipblaslt.md from rocprofv3 CSV output of ``bench.py --probe-contract``
    (one --kernel-trace run and one --pmc run per CONTRACT_PMC_PASSES entry).  Dispatches are told
    apart by kernel family (this build's tm_contract kernels, the library's Cijk kernels); the
    k-th run of consecutive dispatches of a family is the k-th of CONTRACT_SIZES."""
    import collections
    import csv
    mean = lambda xs: sum(xs) / len(xs) if xs else float("nan")

    def family(name):
        return "this build" if "tm_contract" in name else "hipBLASLt" if "Cijk" in name else None

    def runs(rows_in):
        """dispatch id -> (family, N): the k-th run of consecutive dispatches of one family is
        CONTRACT_SIZES[k] (the probe alternates the two families per size)."""
        out, prev, seen = {}, None, collections.Counter()
        for did, name in sorted(rows_in):
            f = family(name)
            if not f:
                continue
            if f != prev:
                seen[f] += 1
                prev = f
            out[did] = (f, CONTRACT_SIZES[min(seen[f], len(CONTRACT_SIZES)) - 1])
        return out

    trace = list(csv.DictReader(open(os.path.join(kt_dir, "run_kernel_trace.csv"))))
    tag = runs({(int(r["Dispatch_Id"]), r["Kernel_Name"]) for r in trace})
    dur = collections.defaultdict(list)
    names = {}
    for r in trace:
        key = tag.get(int(r["Dispatch_Id"]))
        if key:
            dur[key].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
            names[key[0]] = r["Kernel_Name"][:60]
    cnt = collections.defaultdict(lambda: collections.defaultdict(list))
    for d in pmc_dirs:
        pmc = list(csv.DictReader(open(os.path.join(d, "run_counter_collection.csv"))))
        ptag = runs({(int(r["Dispatch_Id"]), r["Kernel_Name"]) for r in pmc})
        for r in pmc:
            key = ptag.get(int(r["Dispatch_Id"]))
            if key:
                cnt[key][r["Counter_Name"]].append(float(r["Counter_Value"]))
    rows = []
    for f in ("this build", "hipBLASLt"):
        for N in CONTRACT_SIZES:
            d, c = dur[(f, N)], cnt[(f, N)]
            if not d:
                continue
            us = mean(d)
            g = lambda k: mean(c[k]) if c.get(k) else float("nan")
            rows.append(dict(f=f, N=N, us=us, tf=2 * N ** 3 * 128 / (us * 1e-6) / 1e12,
                             busy=g("SQ_VALU_MFMA_BUSY_CYCLES") / (128 * g("GRBM_GUI_ACTIVE")),
                             wait=g("SQ_WAIT_INST_ANY") / g("SQ_WAVE_CYCLES"), wany=g("SQ_WAIT_ANY") / g("SQ_WAVE_CYCLES"),
                             lds=g("SQ_INSTS_LDS"), conf=g("SQ_LDS_BANK_CONFLICT"), mfma=g("SQ_INSTS_MFMA"),
                             valu=g("SQ_INSTS_VALU"), salu=g("SQ_INSTS_SALU"), vmem=g("SQ_INSTS_VMEM_RD"),
                             waves=g("SQ_WAVES"), fetch=g("FETCH_SIZE") * 1024))
    cmd = "rocprofv3 --kernel-trace --stats --output-format csv -d <dir> -o run -- python3 bench.py --probe-contract"
    md = ["# Trimul contraction vs hipBLASLt (MI355X, one GPU)", "",
          "Workload: `bench.py --probe-contract`: X = A B^T on [128, N, N] fp16 planes, fp32 accumulation, fp16 "
          "output, 5 launches each of this build's `pf_trimul_contract` and of `torch.bmm` (hipBLASLt, B^T "
          "contiguous) at N = 512, 768, 1024.  Commands (one counter pass each; the table is made by "
          "`bench.py --summarize-contract`):", "", f"    {cmd}"]
    md += [f"    rocprofv3 --pmc {c} --output-format csv -d <dir> -o run -- python3 bench.py --probe-contract"
           for c in CONTRACT_PMC_PASSES]
    md += ["", f"Kernels: this build `{names.get('this build', '?')}`, the library `{names.get('hipBLASLt', '?')}`.",
           "Means per dispatch.  MFMA busy = `SQ_VALU_MFMA_BUSY_CYCLES / (128 GRBM_GUI_ACTIVE)`; wait(inst) = "
           "`SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES` (stalled on s_waitcnt); wait(any) = `SQ_WAIT_ANY / SQ_WAVE_CYCLES`; "
           "FETCH is the raw `FETCH_SIZE` (uncalibrated).", "",
           "| N | kernel | us | TF/s | of 2.5 PF/s | MFMA busy | wait(inst) | wait(any) | waves | MFMA instr | LDS instr "
           "| LDS bank conflict cycles | VALU instr | SALU instr | VMEM rd instr | FETCH MB |",
           "|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for r in sorted(rows, key=lambda r: (r["N"], r["f"] != "this build")):
        md.append(f"| {r['N']} | {r['f']} | {r['us']:.1f} | {r['tf']:.0f} | {r['tf'] / 2500:.3f} | {r['busy']:.3f} | "
                  f"{r['wait']:.2f} | {r['wany']:.2f} | {r['waves']:.0f} | {r['mfma']:.3g} | {r['lds']:.3g} | "
                  f"{r['conf']:.3g} | {r['valu']:.3g} | {r['salu']:.3g} | {r['vmem']:.3g} | {r['fetch'] / 1e6:.0f} |")
    open(os.path.join(ROOT, "profiles", "contract_vs_hipblaslt.md"), "w").write("\n".join(md) + "\n")


def summarize_bench(kt_dir: str, bench_log: str) -> None:
    """profiles/bench_n512_roofline_kernel_stats.txt from a --kernel-trace run of the bench itself
    (``bench.py --no-stack --no-cpu-baseline``) and the JSON line it printed: the in-layer
    attention-core dispatches (those right after a ta_proj dispatch on the same queue, i.e. inside a
    layer) against the line's roofline.launch_ms, the contraction's longest run of back-to-back
    dispatches against roofline_contract.launch_ms, and every kernel of the run."""
    import collections
    import csv
    line = next(json.loads(l) for l in open(bench_log) if l.startswith('{"metric"'))
    rows = sorted(csv.DictReader(open(os.path.join(kt_dir, "run_kernel_trace.csv"))),
                  key=lambda r: int(r["Start_Timestamp"]))
    us = lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    fp16 = lambda r: "DF16_" in r["Kernel_Name"] and "DF16b" not in r["Kernel_Name"]
    prev, inlayer = {}, []
    for r in rows:
        q = r["Queue_Id"]
        k = _kernel_short(r["Kernel_Name"])
        if k == "ta_attn_kernel" and fp16(r) and prev.get(q) == "ta_proj_kernel":
            inlayer.append(us(r))
        prev[q] = k
    best, run, last = [], [], None
    for r in rows:
        k = _kernel_short(r["Kernel_Name"])
        if k == "tm_contract_dma_kernel" and fp16(r) and last == k:
            run.append(us(r))
        elif k == "tm_contract_dma_kernel" and fp16(r):
            run = [us(r)]
        else:
            run = run if k.startswith("__amd") else []
        if len(run) > len(best):
            best = list(run)
        last = k if not k.startswith("__amd") else last
    mean = lambda xs: sum(xs) / len(xs) if xs else float("nan")
    ro, rc = line["roofline"], line["roofline_contract"]
    a_us, c_us = mean(inlayer), mean(best)
    lines = ["# Roofline kernels of the bench, from a kernel trace of the bench itself (MI355X, one GPU)",
             "# command: rocprofv3 --kernel-trace --stats --output-format csv -d <dir> -o run -- python3 bench.py "
             "--no-stack --no-cpu-baseline",
             "# (this file: bench.py --summarize-bench <dir> <the run's stdout>)",
             "# ta_attn_kernel inside the layers: the fp16 dispatches right after a ta_proj dispatch on their queue",
             f"#   {len(inlayer)} dispatches, mean {a_us:.1f} us   | bench roofline.launch_ms = {ro['launch_ms']:.4f} ms "
             f"({ro['launch_ms_source']})",
             f"#   4 N^3 128 FLOP = {ro['flop_per_launch'] / 1e9:.2f} GFLOP / {a_us:.1f} us = "
             f"{ro['flop_per_launch'] / (a_us * 1e-6) / 1e12:.0f} TF/s = "
             f"{ro['flop_per_launch'] / (a_us * 1e-6) / 2.5e15:.3f} of 2.5 PF/s (bench frac {ro['frac']:.4f})",
             f"# tm_contract_dma_kernel: {len(best)} consecutive fp16 dispatches, mean {c_us:.1f} us   | bench "
             f"roofline_contract.launch_ms = {rc['launch_ms']:.4f} ms",
             f"#   {rc['algorithmic_bytes'] / 1e6:.1f} MB / {c_us:.1f} us = {rc['algorithmic_bytes'] / (c_us * 1e3):.0f} "
             f"GB/s = {rc['algorithmic_bytes'] / (c_us * 1e3) / 8000:.3f} of 8 TB/s (bench frac {rc['frac']:.4f})",
             "# Every kernel of the run (warm-up, timed layers, serial layer, per-op breakdown, roofline loops):",
             f"# {'kernel':40s} {'calls':>6s} {'avg_us':>9s} {'total_ms':>9s}"]
    dur = collections.defaultdict(list)
    for r in rows:
        k = _kernel_short(r["Kernel_Name"]) + ("" if fp16(r) or "DF16b" not in r["Kernel_Name"] else " (bf16 lib)")
        dur[k].append(us(r))
    for k, d in sorted(dur.items(), key=lambda kv: -sum(kv[1])):
        if not k.startswith(("distribution", "reduce")):
            lines.append(f"  {k:40s} {len(d):6d} {mean(d):9.1f} {sum(d) / 1e3:9.3f}")
    open(os.path.join(ROOT, "profiles", "bench_n512_roofline_kernel_stats.txt"), "w").write("\n".join(lines) + "\n")


def summarize_stack(kt_dir: str, stack_log: str) -> None:
    """profiles/stack_n768_kernel_stats.txt from a --kernel-trace run of ``bench.py --stack-only``
    and the JSON it printed: the attention core and the 16-bit contraction over every trunk pass
    of the run (warm-up, the four timed passes and the event-timed pass; the contraction's last
    21 dispatches, its warm-up and 20-launch loop alone on random planes, apart) against the
    JSON's attention_in_stack / contract_in_stack and contract, and every kernel of the run."""
    import collections
    import csv
    st = next(json.loads(l) for l in open(stack_log) if l.startswith('{"N"'))
    rows = sorted(csv.DictReader(open(os.path.join(kt_dir, "run_kernel_trace.csv"))),
                  key=lambda r: int(r["Start_Timestamp"]))
    us = lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    mean = lambda xs: sum(xs) / len(xs) if xs else float("nan")
    att = [us(r) for r in rows if _kernel_short(r["Kernel_Name"]) == "ta_attn_kernel"]
    con = [us(r) for r in rows if _kernel_short(r["Kernel_Name"]) == "tm_contract_dma_kernel"]
    con_stack, con_alone = con[:-21], con[-20:]
    N, peak = st["N"], 2.5e15
    f_att, f_con = 4 * N ** 3 * 128, 2 * 128 * N ** 3
    tf = lambda flop, t: flop / (t * 1e-6) / 1e12
    lines = ["# Attention core and trimul contraction inside the config-3 trunk (64 layers, N = 768, MI355X, one GPU)",
             "# command: rocprofv3 --kernel-trace --stats --output-format csv -d <dir> -o run -- python3 bench.py --stack-only",
             "# (this file: bench.py --summarize-stack <dir> <the run's stdout>)",
             f"# trunk: {st['layers_per_s']} layers/s ({st['trunk_s']} s for {st['passes']} passes) in that run",
             f"# ta_attn_kernel: {len(att)} dispatches, mean {mean(att):.1f} us = {tf(f_att, mean(att)):.0f} TF/s = "
             f"{tf(f_att, mean(att)) * 1e12 / peak:.3f} of 2.5 PF/s   | attention_in_stack "
             f"{st['attention_in_stack']['launch_ms'] * 1e3:.1f} us (HIP events)",
             f"# tm_contract_dma_kernel in the trunk: {len(con_stack)} dispatches, mean {mean(con_stack):.1f} us = "
             f"{tf(f_con, mean(con_stack)):.0f} TF/s = {tf(f_con, mean(con_stack)) * 1e12 / peak:.3f}   | "
             f"contract_in_stack {st['contract_in_stack']['launch_ms'] * 1e3:.1f} us (HIP events)",
             f"# tm_contract_dma_kernel alone (random planes): {len(con_alone)} dispatches, mean {mean(con_alone):.1f} us = "
             f"{tf(f_con, mean(con_alone)):.0f} TF/s = {tf(f_con, mean(con_alone)) * 1e12 / peak:.3f}   | "
             f"contract {st['contract']['launch_ms'] * 1e3:.1f} us",
             "# Every kernel of the run:",
             f"# {'kernel':40s} {'calls':>6s} {'avg_us':>9s} {'total_ms':>9s}"]
    dur = collections.defaultdict(list)
    for r in rows:
        dur[_kernel_short(r["Kernel_Name"])].append(us(r))
    for k, d in sorted(dur.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"  {k:40s} {len(d):6d} {mean(d):9.1f} {sum(d) / 1e3:9.3f}")
    open(os.path.join(ROOT, "profiles", "stack_n768_kernel_stats.txt"), "w").write("\n".join(lines) + "\n")


# ----------------------------------------------------------------------------- profile summaries
PROBE_PMC_PASSES = ("SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS "
                    "SQ_VALU_MFMA_BUSY_CYCLES SQ_WAIT_INST_ANY GRBM_GUI_ACTIVE",
                    "FETCH_SIZE GRBM_GUI_ACTIVE", "WRITE_SIZE GRBM_GUI_ACTIVE")


def _kernel_short(name: str) -> str:
    import re
    m = re.search(r"N_\d+([a-z0-9_]+_kernel)|([a-z0-9_]+_kernel)", name)
    k = (m.group(1) or m.group(2)) if m else name[:40]
    if k == "tr_pair_kernel" and ("Li3E" in name or ", 3>" in name):
        return "tr_pair_kernel (fc3 sampling pass)"
    return "copy (torch.mul, calibration)" if "MulFunctor" in name else k


def summarize_probe(N: int, kt_dir: str, pmc_dirs) -> None:
    """Write profiles/layer_n{N}_kernel_stats.txt, profiles/layer_n{N}_counters.md and (N = 512)
    profiles/kernel_traffic_n512.json from rocprofv3 CSV output of ``bench.py --probe-traffic
    --n N``: one --kernel-trace run (``kt_dir``) and one --pmc run per PROBE_PMC_PASSES entry
    (``pmc_dirs``), each written with ``--output-format csv -o run``."""
    import collections
    import csv
    mean = lambda xs: sum(xs) / len(xs) if xs else float("nan")
    dur = collections.defaultdict(list)
    for r in csv.DictReader(open(os.path.join(kt_dir, "run_kernel_trace.csv"))):
        dur[_kernel_short(r["Kernel_Name"])].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    cnt = collections.defaultdict(lambda: collections.defaultdict(list))
    for d in pmc_dirs:
        for r in csv.DictReader(open(os.path.join(d, "run_counter_collection.csv"))):
            k, v = _kernel_short(r["Kernel_Name"]), float(r["Counter_Value"])
            if k.startswith("copy") and r["Counter_Name"] in ("FETCH_SIZE", "WRITE_SIZE") and v < 100 * 1024:
                continue   # small torch.mul calls elsewhere in the probe are not the calibration copy
            cnt[k][r["Counter_Name"]].append(v)
    copy = cnt["copy (torch.mul, calibration)"]
    f_fac = COPY_BYTES / (mean(copy["FETCH_SIZE"]) * 1024)
    w_fac = COPY_BYTES / (mean(copy["WRITE_SIZE"]) * 1024)
    copy_us = mean([d for d in dur["copy (torch.mul, calibration)"] if d > 20])
    P = N * N
    alg = {"tm_proj_kernel": P * 128 * 4 + 2 * P * 128 * 2,
           "tm_contract_dma_kernel": 3 * P * 128 * 2,
           "tm_out_kernel": P * 128 * 2 + 2 * P * 128 * 4,
           "ta_proj_kernel": P * 128 * 4 + 3 * P * 128 * 2 + 4 * P * 4 + P * 2,
           "ta_attn_kernel": 3 * P * 128 * 2 + 4 * P * 4 + P * 2 + P * 128 * 2,
           "ta_out_kernel": P * 128 * 2 + 2 * P * 128 * 4,
           "tr_pair_kernel": 2 * P * 128 * 4 + 16 * P * 4}
    rows = []
    for k in sorted(cnt, key=lambda k: -sum(dur.get(k, [0]))):
        c, d = cnt[k], dur.get(k, [])
        if not d or k.startswith(("distribution", "reduce", "__amd")):
            continue
        fe = mean(c["FETCH_SIZE"]) * 1024 * f_fac if c.get("FETCH_SIZE") else float("nan")
        wr = mean(c["WRITE_SIZE"]) * 1024 * w_fac if c.get("WRITE_SIZE") else float("nan")
        gr = mean(c["GRBM_GUI_ACTIVE"])
        us = mean(d)
        rows.append(dict(kernel=k, us=us, fetch=fe, write=wr, gbs=(fe + wr) / (us * 1e3), alg=alg.get(k),
                         mfma=mean(c["SQ_INSTS_MFMA"]) if c.get("SQ_INSTS_MFMA") else 0.0,
                         busy=mean(c["SQ_VALU_MFMA_BUSY_CYCLES"]) / (128 * gr) if c.get("SQ_VALU_MFMA_BUSY_CYCLES")
                         else float("nan"),
                         valu=mean(c["SQ_INSTS_VALU"]) if c.get("SQ_INSTS_VALU") else float("nan"),
                         wait=mean(c["SQ_WAIT_INST_ANY"]) / mean(c["SQ_WAVE_CYCLES"]) if c.get("SQ_WAIT_INST_ANY")
                         else float("nan")))
    cmd_kt = (f"rocprofv3 --kernel-trace --stats --output-format csv -d <dir> -o run -- python3 bench.py "
              f"--probe-traffic --n {N}")
    lines = [f"# Kernel durations, bench.py --probe-traffic at N={N} (MI355X, one GPU)", f"# command: {cmd_kt}",
             "# workload: the triangle-attention core x5 and the trimul contraction x5 on their real operands,",
             "# a 256 MiB copy x3 (calibration), then 3 full PairformerLayers (serial schedule, single track included)",
             f"# {'kernel':34s} {'calls':>6s} {'avg_us':>9s} {'total_ms':>9s}"]
    for k, d in sorted(dur.items(), key=lambda kv: -sum(kv[1])):
        if not k.startswith(("distribution", "__amd", "reduce")):
            lines.append(f"  {k:34s} {len(d):6d} {mean(d):9.1f} {sum(d) / 1e3:9.3f}")
    open(os.path.join(ROOT, "profiles", f"layer_n{N}_kernel_stats.txt"), "w").write("\n".join(lines) + "\n")
    md = [f"# Per-kernel counters, N = {N} (MI355X, one GPU)", "",
          f"Workload: `bench.py --probe-traffic --n {N}` (attention core x5, trimul contraction x5, a 256 MiB copy x3 "
          "for calibration, three full PairformerLayers).  Commands (one counter pass each; durations from the kernel "
          "trace; the tables are made by `bench.py --summarize-probe`):", "", f"    {cmd_kt}"]
    md += [f"    rocprofv3 --pmc {c} --output-format csv -d <dir> -o run -- python3 bench.py --probe-traffic --n {N}"
           for c in PROBE_PMC_PASSES]
    md += ["", "Values are means per dispatch over every dispatch of the kernel in the run.",
           f"HBM bytes: `FETCH_SIZE` x {f_fac:.3f} and `WRITE_SIZE` x {w_fac:.3f} (KiB): the factors that make the "
           f"plain copy kernel's counters read its known 256 MiB in / 256 MiB out (the copy itself ran at "
           f"{2 * COPY_BYTES / (copy_us * 1e3):.0f} GB/s).",
           "MFMA busy = `SQ_VALU_MFMA_BUSY_CYCLES / (128 GRBM_GUI_ACTIVE)` (GRBM summed over the 8 XCDs, 1024 SIMDs).",
           "wait = `SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES` (fraction of wave time stalled on s_waitcnt).", "",
           "MFMA TF/s = issued `SQ_INSTS_MFMA` x 32768 FLOP (one 32x32x16 f16 MFMA) per second.", "",
           "| kernel | us | HBM read MB | HBM write MB | GB/s | of 8 TB/s | algorithmic MB | traffic / algorithmic "
           "| MFMA instr | MFMA busy | MFMA TF/s | VALU instr | wait |",
           "|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for r in rows:
        ratio = (r["fetch"] + r["write"]) / r["alg"] if r["alg"] else float("nan")
        tf = r["mfma"] * 32768 / (r["us"] * 1e-6) / 1e12
        md.append(f"| {r['kernel']} | {r['us']:.1f} | {r['fetch'] / 1e6:.1f} | {r['write'] / 1e6:.1f} | "
                  f"{r['gbs']:.0f} | {r['gbs'] / 8000:.2f} | {(r['alg'] or float('nan')) / 1e6:.1f} | {ratio:.2f} | "
                  f"{r['mfma']:.0f} | {r['busy']:.3f} | {tf:.0f} | {r['valu']:.3g} | {r['wait']:.2f} |")
    open(os.path.join(ROOT, "profiles", f"layer_n{N}_counters.md"), "w").write("\n".join(md) + "\n")
    if N == 512:
        t = {"N": N, "note": ("HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE over bench.py "
                              f"--probe-traffic (mean per dispatch, scaled by {f_fac:.3f} / {w_fac:.3f}: the factors "
                              "that make a plain 256 MiB copy read its known bytes); VALU and MFMA instructions per "
                              "launch from SQ_INSTS_VALU / SQ_INSTS_MFMA"),
             "kernels": {r["kernel"]: {"hbm_bytes_per_launch": round(r["fetch"] + r["write"]),
                                        "read_bytes": round(r["fetch"]), "write_bytes": round(r["write"]),
                                        "algorithmic_bytes": r["alg"], "launch_us": round(r["us"], 1),
                                        "valu_instr_per_launch": round(r["valu"]),
                                        "mfma_instr_per_launch": round(r["mfma"])}
                         for r in rows if r["alg"]}}
        json.dump(t, open(TRAFFIC_FILE, "w"), indent=1)


def load_traffic():
    """Calibrated HBM bytes per launch of the roofline kernels from the committed PMC summary
    (``{"N": .., "note": .., "kernels": {name: {"hbm_bytes_per_launch": ..}}}``, or None)."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return t
    except (OSError, ValueError):
        return None


#: Issue cost of one wave64 VALU instruction per SIMD on this chip under load (ns), from in-bounds
#: throughput microbenchmarks (8 waves per SIMD): v_exp_f32 (transcendental, quarter rate) and
#: v_fma_f32 (every other 32-bit VALU instruction is priced at the FMA rate).
VALU_NS = {"v_exp_f32": 3.74, "other": 2.12}


def valu_roof(kname: str, N: int, launch_ms: float, simds: int, counters_for) -> Optional[dict]:
    """The VALU / transcendental roof of the attention core: its VALU instructions per launch
    (SQ_INSTS_VALU from the committed PMC summary) priced at the measured issue costs, one v_exp_f32
    per score (N^3 * 4 heads, 64 per wave instruction), spread over every SIMD: the time the VALU
    pipe alone needs, and its fraction of the launch time."""
    k = counters_for(kname)
    if not k or not k.get("valu_instr_per_launch"):
        return None
    valu = float(k["valu_instr_per_launch"])
    exp_instr = N ** 3 * 4 / 64
    floor_ns = (exp_instr * VALU_NS["v_exp_f32"] + max(valu - exp_instr, 0.0) * VALU_NS["other"]) / simds
    return {"bound": "valu", "instructions_per_launch": valu, "exp_instructions_per_launch": exp_instr,
            "issue_ns_per_wave_instr": VALU_NS, "simds": simds, "floor_ms": round(floor_ns * 1e-6, 4),
            "frac": round(floor_ns * 1e-6 / launch_ms, 4),
            "note": "floor = the VALU pipe's issue time for this launch's instruction count (counters: "
                    "profiles/kernel_traffic_n%d.json); frac = floor / in-layer launch time" % N}


def time_events(fn, reps: int, stream) -> float:
    """Average ms per call of fn, HIP events recorded on `stream` (the stream the kernels use)."""
    import torch
    fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        fn()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def contract_vs_library(reps: int = 10) -> dict:
    """The 16-bit trimul contraction X = A B^T on [128, N, N] fp16 planes against torch.bmm
    (hipBLASLt; B^T contiguous) at N = 512, 768, 1024, HIP events around `reps` launches each on
    the current stream; TF/s = 2 N^3 128 / time."""
    import torch
    from tt_boltz_amd import ops
    dev, stream = torch.device("cuda", 0), torch.cuda.current_stream()
    g = torch.Generator(device=dev).manual_seed(0)
    res = {}
    for N in CONTRACT_SIZES:
        A = torch.randn((128, N, N), device=dev, generator=g).half()
        Bm = torch.randn((128, N, N), device=dev, generator=g).half()
        Bt = Bm.transpose(1, 2).contiguous()
        X = torch.empty((128, N, N), dtype=torch.float16, device=dev)
        ours = time_events(lambda: ops.launch_trimul_contract(A, Bm, X), reps, stream)
        lib = time_events(lambda: torch.bmm(A, Bt, out=X), reps, stream)
        tf = lambda ms: round(2 * N ** 3 * 128 / (ms * 1e-3) / 1e12, 1)
        res[str(N)] = {"this_build_ms": round(ours, 4), "hipblaslt_ms": round(lib, 4), "this_build_tflops": tf(ours),
                       "hipblaslt_tflops": tf(lib), "speedup": round(lib / ours, 3)}
        del A, Bm, Bt, X
        torch.cuda.empty_cache()
    res["note"] = ("pf_trimul_contract (fp16 output) vs torch.bmm(A, B^T) on the same random fp16 planes, fp32 "
                   "accumulation; counters side by side in profiles/contract_vs_hipblaslt.md")
    return res


def stack_bench(N: int = 768, n_layers: int = 64, recycling_steps: int = 3, seed: int = 3) -> dict:
    """Config 3: the 64-layer trunk at N=768 through the device-resident recycling loop
    (boltz2.py:5203-5248; recycling_steps=3 -> 4 passes), plus the contraction alone at N."""
    import torch
    from tt_boltz_amd import ops, pairformer, synthetic
    dev = pairformer.get_device()
    stream = torch.cuda.current_stream()
    w = synthetic.stack_weights(n_layers, seed)
    w_rec = synthetic.draw(synthetic.recycle_shapes(), seed + 1000)
    s_cpu, z_cpu, mask_cpu, _ = synthetic.pair_inputs(N, seed, z_scale=0.5)
    pf = pairformer.Pairformer(n_layers, 32, 4, 24, 16, True, w)
    rec = pairformer.TrunkRecycler(pf, w_rec)
    s0, z0, mask = s_cpu.to(dev), z_cpu.to(dev), mask_cpu.to(dev)
    rec(s0, z0, mask, 0)            # warm-up pass
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    s_out, z_out = rec(s0, z0, mask, recycling_steps)
    e1.record(stream)
    torch.cuda.synchronize()
    trunk_s = e0.elapsed_time(e1) / 1e3
    finite = bool(torch.isfinite(z_out).all() and torch.isfinite(s_out).all())
    passes = recycling_steps + 1
    fl = flops_layer(N)
    # one more pass with HIP events around every launch of the attention core and of the 16-bit
    # contraction (on the pair stream, as in the timed passes): their in-stack launch times
    ops.kernel_timing(ops.TIMED_ATTEND, True)
    ops.kernel_timing(ops.TIMED_CONTRACT, True)
    rec(s0, z0, mask, 0)
    att_ms, att_n = ops.kernel_timing_read(ops.TIMED_ATTEND)
    con_ms, con_n = ops.kernel_timing_read(ops.TIMED_CONTRACT)
    ops.kernel_timing(ops.TIMED_ATTEND, False)
    ops.kernel_timing(ops.TIMED_CONTRACT, False)
    torch.cuda.synchronize()

    def in_stack(total_ms, n, flop):
        ms = total_ms / max(n, 1)
        tf = flop / (ms * 1e-3) / 1e12
        return {"launch_ms": round(ms, 4), "launches": n, "tflops": round(tf, 1),
                "frac_of_peak": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)}
    # the contraction alone at this N (128 planes, one direction per launch)
    A = torch.randn((128, N, N), device=dev).half()
    Bm = torch.randn((128, N, N), device=dev).half()
    X = torch.empty((128, N, N), dtype=torch.float16, device=dev)
    c_ms = time_events(lambda: ops.launch_trimul_contract(A, Bm, X), 20, stream)
    c_tf = fl["trimul_contract"] / (c_ms * 1e-3) / 1e12
    del A, Bm, X
    return {"N": N, "layers": n_layers, "recycling_steps": recycling_steps, "passes": passes,
            "trunk_s": round(trunk_s, 4), "pass_s": round(trunk_s / passes, 4),
            "layers_per_s": round(n_layers * passes / trunk_s, 2),
            "layer_tflops_achieved": round(fl["layer"] * n_layers * passes / trunk_s / 1e12, 1),
            "finite": finite,
            "contract": {"kernel": "tm_contract_dma_kernel", "launch_ms": round(c_ms, 4),
                         "tflops": round(c_tf, 1), "frac_of_peak": round(c_tf / MFMA_BF16_PEAK_TFLOPS, 4),
                         "note": "alone: 20 back-to-back launches on random [128, N, N] fp16 planes"},
            "contract_in_stack": {"kernel": "tm_contract_dma_kernel", **in_stack(con_ms, con_n, fl["trimul_contract"]),
                                  "note": "HIP events around each launch during one extra 64-layer pass"},
            "attention_in_stack": {"kernel": "ta_attn_kernel", **in_stack(att_ms, att_n, fl["triatt_core"]),
                                   "note": "HIP events around each launch during one extra 64-layer pass"},
            "workload": "64-layer Boltz-2 Pairformer trunk, N=768, seed 3 weights, z~0.5 N(0,1), s~N(0,1), "
                        "masks all ones, 4 recycling passes, fp32 residual stream"}


def msa_bench(N: int = 512, S: int = 1024, seed: int = 5, steps: int = 3) -> dict:
    """One MSA layer of the Boltz-2 MSA module (the next row after the Pairformer): pair
    weighted averaging, MSA transition, outer product mean and the no-seq PairformerLayer,
    at N tokens and S MSA rows, masks all ones; each op timed alone and the layer."""
    import torch
    from tt_boltz_amd import msa as msa_mod, ops, pairformer, synthetic
    dev = pairformer.get_device()
    stream = torch.cuda.current_stream()
    w = synthetic.draw(synthetic.msa_layer_shapes(), seed)
    layer = msa_mod.MSALayer(32, 8, 32, 4, w)
    g = torch.Generator().manual_seed(seed)
    z = torch.randn((1, N, N, 128), generator=g).to(dev).contiguous()
    m = torch.randn((1, S, N, 64), generator=g).to(dev).contiguous()
    ws = ops.workspace(layer.workspace_bytes(1, S, N), dev)
    ms = {
        "pair_weighted_averaging": time_events(lambda: layer.pair_weighted_averaging(m, z, None, ws), steps, stream),
        "msa_transition": time_events(lambda: layer.msa_transition(m, out=m, accumulate=True, ws=ws), steps, stream),
        "outer_product_mean": time_events(lambda: layer.outer_product_mean(m, None, z, ws), steps, stream),
        "pairformer_noseq_layer": time_events(lambda: layer.pairformer_layer(None, z, None, None, ws), steps, stream),
        "layer": time_events(lambda: layer(z, m, None, None, ws), steps, stream),
    }
    opm_fl = 2 * (32 * N) ** 2 * S + 2 * N * N * 1024 * 128
    pwa_fl = 2 * N * N * S * 256
    return {"N": N, "S": S, "seed": seed, "layer_ms": round(ms["layer"], 3),
            "layers_per_s": round(1000.0 / ms["layer"], 2),
            "ops_ms": {k: round(v, 3) for k, v in ms.items() if k != "layer"},
            "outer_product_mean_tflops": round(opm_fl / (ms["outer_product_mean"] * 1e-3) / 1e12, 1),
            "pair_weighted_averaging_tflops": round(pwa_fl / (ms["pair_weighted_averaging"] * 1e-3) / 1e12, 1),
            "finite": bool(torch.isfinite(z).all() and torch.isfinite(m).all()),
            "workload": f"one Boltz-2 MSALayer, N={N} tokens, S={S} MSA rows, c_m=64, PWA 8x32, OPM hidden 32, "
                        "masks all ones, seed 5 weights"}


def diffusion_bench(N: int = 512, depth: int = 24, heads: int = 16, seed: int = 6, steps: int = 5) -> dict:
    """Pair side of the diffusion conditioning at N tokens: PairwiseConditioning (projection
    of cat(z, rel_pos) + 2 transitions) and the token-transformer pair bias (depth x heads
    outputs per pair), each timed alone; the bias kernel's HBM rate against its algorithmic
    bytes (z read once, the bias written once, fp32)."""
    import torch
    from tt_boltz_amd import diffusion, pairformer, synthetic
    dev = pairformer.get_device()
    stream = torch.cuda.current_stream()
    w = synthetic.draw(synthetic.diffusion_pair_shapes(depth=depth, heads=heads), seed)
    cond = diffusion.PairwiseConditioning(pairformer.WeightScope.wrap(w).child("pairwise_conditioner"))
    bias = diffusion.TokenTransformerPairBias(depth, w)
    g = torch.Generator().manual_seed(seed)
    zt = torch.randn((1, N, N, 128), generator=g).to(dev).contiguous()
    rp = torch.randn((1, N, N, 128), generator=g).to(dev).contiguous()
    z = torch.empty_like(zt)
    M = depth * heads
    out0 = torch.empty((1, N, N, M), dtype=torch.float32, device=dev)
    out1 = torch.empty((M, 1, N, N), dtype=torch.float32, device=dev)
    ms_cond = time_events(lambda: cond(zt, rp, out=z), steps, stream)
    ms_b0 = time_events(lambda: bias(z, 0, 1.0, out0), steps, stream)
    ms_b1 = time_events(lambda: bias(z, 1, 1.0, out1), steps, stream)
    nbytes = N * N * (128 + M) * 4
    return {"N": N, "depth": depth, "heads": heads, "pairwise_conditioning_ms": round(ms_cond, 3),
            "token_bias_ms": round(ms_b0, 3), "token_bias_head_major_ms": round(ms_b1, 3),
            "token_bias_algorithmic_bytes": nbytes, "token_bias_TBps": round(nbytes / (ms_b0 * 1e-3) / 1e12, 2),
            "token_bias_head_major_TBps": round(nbytes / (ms_b1 * 1e-3) / 1e12, 2),
            "finite": bool(torch.isfinite(out0).all() and torch.isfinite(z).all())}


def template_bench(N: int = 512, T: int = 4, seed: int = 7, steps: int = 5) -> dict:
    """The template stack's Pairformer (2 no-seq layers at c_z = 64, boltz2.py:3748-3761) on
    T templates (the batch the template module runs it on) at N tokens: ms per 2-layer pass
    and per layer, masks all ones."""
    import torch
    from tt_boltz_amd import ops, pairformer, synthetic
    dev = pairformer.get_device()
    stream = torch.cuda.current_stream()
    w = synthetic.stack_weights(2, seed, c_z=64, transform_s=False)
    pf = pairformer.Pairformer(2, 32, 4, None, None, False, w)
    z = torch.randn((T, N, N, 64), generator=torch.Generator().manual_seed(seed)).to(dev).contiguous()
    ws = ops.workspace(pf.workspace_bytes(T, N), dev)
    ms = time_events(lambda: pf(None, z, None, None, ws), steps, stream)
    layer = pf.blocks[0]
    ops_ms = {
        "trimul_out": time_events(lambda: layer.triangle_multiplication_start(z, None, out=z, accumulate=True, ws=ws),
                                  steps, stream),
        "triatt_start": time_events(lambda: layer.triangle_attention_start(z, None, out=z, accumulate=True, ws=ws),
                                    steps, stream),
        "transition_z": time_events(lambda: layer.transition_z(z, out=z, accumulate=True, ws=ws), steps, stream),
    }
    return {"N": N, "templates": T, "c_z": 64, "stack_ms": round(ms, 3), "layer_ms": round(ms / 2, 3),
            "template_layers_per_s": round(2000.0 / ms, 2), "ops_ms": {k: round(v, 3) for k, v in ops_ms.items()},
            "finite": bool(torch.isfinite(z).all())}


def msa_trunk_bench(N: int = 768, S: int = 1024, msa_blocks: int = 4, n_layers: int = 64, recycling_steps: int = 3,
                    seed: int = 8) -> dict:
    """The trunk loop with the MSA module on the device: each of the 4 passes runs the
    recycling projections, z = z + MSA(z) (4 MSA blocks over S sequences) and the 64-layer
    Pairformer (boltz2.py:5203-5248), nothing leaving the GPU; reported next to the same loop
    without the MSA module (the stack object)."""
    import torch
    from tt_boltz_amd import msa as msa_mod, pairformer, synthetic
    dev = pairformer.get_device()
    stream = torch.cuda.current_stream()
    w = synthetic.stack_weights(n_layers, seed)
    w_rec = synthetic.draw(synthetic.recycle_shapes(), seed + 1000)
    w_msa = synthetic.draw(synthetic.msa_module_shapes(msa_blocks), seed + 2000)
    s_cpu, z_cpu, mask_cpu, _ = synthetic.pair_inputs(N, seed, z_scale=0.5)
    g = torch.Generator().manual_seed(seed)
    feats = {"msa": torch.randint(0, msa_mod.NUM_TOKENS, (1, S, N), generator=g),
             "has_deletion": (torch.rand((1, S, N), generator=g) > 0.8).float(),
             "deletion_value": torch.rand((1, S, N), generator=g),
             "msa_paired": (torch.rand((1, S, N), generator=g) > 0.5).float(),
             "msa_mask": torch.ones((1, S, N))}
    emb = torch.randn((1, N, 384), generator=g)
    pf = pairformer.Pairformer(n_layers, 32, 4, 24, 16, True, w)
    rec = pairformer.TrunkRecycler(pf, w_rec, msa=msa_mod.MSA(msa_blocks, 32, 8, 32, 4, w_msa))
    inputs = msa_mod.device_inputs(emb, feats, N, dev)
    s0, z0, mask = s_cpu.to(dev), z_cpu.to(dev), mask_cpu.to(dev)
    rec(s0, z0, mask, 0, msa_inputs=inputs)   # warm-up pass
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    s_out, z_out = rec(s0, z0, mask, recycling_steps, msa_inputs=inputs)
    e1.record(stream)
    torch.cuda.synchronize()
    trunk_s = e0.elapsed_time(e1) / 1e3
    passes = recycling_steps + 1
    return {"N": N, "S": S, "msa_blocks": msa_blocks, "layers": n_layers, "passes": passes,
            "trunk_s": round(trunk_s, 4), "pass_s": round(trunk_s / passes, 4),
            "finite": bool(torch.isfinite(z_out).all() and torch.isfinite(s_out).all()),
            "workload": f"Boltz-2 trunk with the MSA module on the device: {msa_blocks} MSA blocks over S={S} "
                        f"sequences + {n_layers} Pairformer layers per pass, N={N}, {passes} passes, masks all ones"}


def module_bench(N: int = 512, n_layers: int = 4, seed: int = 9, reps: int = 3) -> dict:
    """The drop-in PairformerModule on CPU tensors (as tt-bio calls it): padding, H2D of s/z,
    n_layers layers, D2H of the outputs, timed with the host clock around forward (second
    call onwards, masks cached), next to the same layers on device-resident tensors."""
    import torch
    from tt_boltz_amd import pairformer, synthetic
    dev = pairformer.get_device()
    w = synthetic.stack_weights(n_layers, seed)
    s, z, mask, pm = synthetic.pair_inputs(N, seed)
    mod = pairformer.PairformerModule(n_layers, 32, 4, 24, 16, True)
    mod.load_state_dict(w)
    mod(s, z, mask=mask, pair_mask=pm)
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        s_out, z_out = mod(s, z, mask=mask, pair_mask=pm)
        ts.append(time.perf_counter() - t0)
    e2e = sorted(ts)[len(ts) // 2]
    sd, zd, md, pmd = s.to(dev), z.to(dev), mask.to(dev), pm.to(dev).contiguous()
    pf = mod.module
    pf(sd.clone(), zd.clone(), pmd, md)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        pf(sd.clone(), zd.clone(), pmd, md)
    torch.cuda.synchronize()
    dev_s = (time.perf_counter() - t0) / reps
    return {"N": N, "layers": n_layers, "end_to_end_s": round(e2e, 4), "device_resident_s": round(dev_s, 4),
            "host_copy_overhead_s": round(e2e - dev_s, 4),
            "end_to_end_layers_per_s": round(n_layers / e2e, 1),
            "note": "PairformerModule.forward on CPU fp32 tensors (pad, H2D, layers, D2H; PCIe-inclusive) vs the "
                    "device-resident stack on the same inputs; host clock, median of 3"}


def fast_bench(N: int = 1024, seed: int = 4, steps: int = 5) -> dict:
    """Config 4: one layer in fast mode (MXFP8 triangle multiplications and pair
    transition) at N=1024 next to the same layer in 16-bit, plus the fp8 contraction alone."""
    import torch
    from tt_boltz_amd import ops, pairformer, synthetic
    dev = pairformer.get_device()
    stream = torch.cuda.current_stream()
    w = synthetic.stack_weights(1, seed)
    s_cpu, z_cpu, _, _ = synthetic.pair_inputs(N, seed)
    res = {"N": N, "seed": seed}
    for mode in ("fp8", "fp16"):
        pairformer.set_fast_mode(mode == "fp8")
        try:
            pf = pairformer.Pairformer(1, 32, 4, 24, 16, True, w)
        finally:
            pairformer.set_fast_mode(False)
        ws = ops.workspace(pf.workspace_bytes(1, N), dev)
        z, s = z_cpu.to(dev).contiguous(), s_cpu.to(dev).contiguous()
        layer = pf.blocks[0]
        layer(s, z, None, None, ws)
        torch.cuda.synchronize()
        if mode == "fp8":   # the contraction's own launches inside the timed layers
            ops.kernel_timing(ops.TIMED_CONTRACT8, True)
        ms = time_events(lambda: layer(s, z, None, None, ws), steps, stream)
        if mode == "fp8":
            c_total, c_n = ops.kernel_timing_read(ops.TIMED_CONTRACT8)
            ops.kernel_timing(ops.TIMED_CONTRACT8, False)
            c_in = c_total / max(c_n, 1)
        res[f"{mode}_layer_ms"] = round(ms, 3)
        res[f"{mode}_layers_per_s"] = round(1000.0 / ms, 2)
        tm = layer.triangle_multiplication_start
        res[f"{mode}_trimul_ms"] = round(time_events(lambda: tm(z, None, out=z, accumulate=True, ws=ws), steps,
                                                     stream), 3)
        del pf, ws, z, s, layer, tm
    torch.cuda.empty_cache()
    # the MXFP8 contraction alone: 128 planes, fp32 output (the standalone entry point)
    g = torch.Generator(device=dev).manual_seed(seed)
    qa, sa = ops.quantize_mx8(torch.randn((128 * N, N), device=dev, generator=g))
    qb, sb = ops.quantize_mx8(torch.randn((128 * N, N), device=dev, generator=g))
    X = torch.empty((128, N, N), dtype=torch.float32, device=dev)
    c_ms = time_events(lambda: ops.launch_trimul_mx8_contract(qa.view(128, N, N), qb.view(128, N, N),
                                                              sa.view(128, N, N // 32), sb.view(128, N, N // 32), X),
                       10, stream)
    tf = 2 * N ** 3 * 128 / (c_ms * 1e-3) / 1e12
    tf_in = 2 * N ** 3 * 128 / (c_in * 1e-3) / 1e12
    peak8 = ops.mfma_rate_probe(dev, fp8=True)
    res["mx8_contract"] = {"kernel": "tm8_contract_kernel", "launch_ms": round(c_in, 4), "tflops": round(tf_in, 1),
                           "peak_fp8_tflops": 5000.0, "frac_of_fp8_peak": round(tf_in / 5000.0, 4),
                           "launch_ms_source": f"in-layer: mean of {c_n} launches inside the fp8 layers of the line (the timed steps and one warm-up step) "
                                               "(HIP events; fp16 output, as the trimul writes it)",
                           "measured_peak_fp8": {**peak8, "frac": round(tf_in / peak8["tflops"], 4),
                                                 "note": "sustained block-scaled fp8 MFMA rate under load "
                                                         "(mfma8_rate_kernel, random e4m3 operands)"},
                           "standalone_fp32_out": {"launch_ms": round(c_ms, 4), "tflops": round(tf, 1),
                                                   "note": "pf_trimul_mx8_contract (fp32 output: 512 MB written "
                                                           "per launch at N=1024)"}}
    res["error_vs_fp32"] = ("measured by tests/test_gpu_fast.py at N=1024 (mean / max of the fp32 result's rms): "
                            "trimul update 5.7e-2 / 0.71, pair transition 5.2e-2 / 0.41, whole fast layer z "
                            "4.4e-2 / 0.50 (1.8e-2 mean from the emulated-fp8 layer)")
    return res


def fast_trunk_bench(N: int = 1024, n_layers: int = 64, seed: int = 4) -> dict:
    """Config 4 as a trunk: one pass of the 64-layer Pairformer stack at N=1024 in fast mode
    (every block-fp8 point) next to the same stack in 16-bit, device-resident, masks all ones;
    each after one untimed pass."""
    import torch
    from tt_boltz_amd import ops, pairformer, synthetic
    dev = pairformer.get_device()
    stream = torch.cuda.current_stream()
    w = synthetic.stack_weights(n_layers, seed)
    s_cpu, z_cpu, mask_cpu, _ = synthetic.pair_inputs(N, seed)
    res = {"N": N, "layers": n_layers, "seed": seed}
    for mode in ("fp8", "fp16"):
        pairformer.set_fast_mode(mode == "fp8")
        try:
            pf = pairformer.Pairformer(n_layers, 32, 4, 24, 16, True, w)
        finally:
            pairformer.set_fast_mode(False)
        ws = ops.workspace(pf.workspace_bytes(1, N), dev)
        z, s, mask = z_cpu.to(dev).contiguous(), s_cpu.to(dev).contiguous(), mask_cpu.to(dev)
        pf(s.clone(), z.clone(), None, mask, ws)   # untimed pass
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        s_out, z_out = pf(s, z, None, mask, ws)
        e1.record(stream)
        torch.cuda.synchronize()
        sec = e0.elapsed_time(e1) / 1e3
        res[f"{mode}_pass_s"] = round(sec, 4)
        res[f"{mode}_layers_per_s"] = round(n_layers / sec, 2)
        res[f"{mode}_finite"] = bool(torch.isfinite(z_out).all() and torch.isfinite(s_out).all())
        del pf, ws, z, s, mask, s_out, z_out
        torch.cuda.empty_cache()
    res["speedup"] = round(res["fp16_pass_s"] / res["fp8_pass_s"], 3)
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--n", type=int, default=512)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-stack", action="store_true")
    ap.add_argument("--probe-traffic", action="store_true")
    ap.add_argument("--probe-contract", action="store_true")
    ap.add_argument("--summarize-bench", nargs=2, metavar=("KT_DIR", "BENCH_LOG"),
                    help="write profiles/bench_n512_roofline_kernel_stats.txt from a kernel trace of the bench")
    ap.add_argument("--summarize-contract", nargs="+", metavar="DIR",
                    help="KT_DIR PMC_DIR...: write profiles/contract_vs_hipblaslt.md from rocprofv3 CSV output")
    ap.add_argument("--stack-only", action="store_true",
                    help="print only the config-3 trunk object (stack_bench) as JSON")
    ap.add_argument("--summarize-stack", nargs=2, metavar=("KT_DIR", "STACK_LOG"),
                    help="write profiles/stack_n768_kernel_stats.txt from a kernel trace of --stack-only")
    ap.add_argument("--summarize-probe", nargs="+", metavar="DIR",
                    help="KT_DIR PMC_DIR...: write the profiles/ summaries for --n from rocprofv3 CSV output")
    args = ap.parse_args()
    if args.summarize_probe:
        summarize_probe(args.n, args.summarize_probe[0], args.summarize_probe[1:])
        return 0
    if args.summarize_bench:
        summarize_bench(*args.summarize_bench)
        return 0
    if args.summarize_contract:
        summarize_contract(args.summarize_contract[0], args.summarize_contract[1:])
        return 0
    if args.summarize_stack:
        summarize_stack(*args.summarize_stack)
        return 0
    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU (got --gpus {args.gpus}): this build measures the "
              "single-GPU Pairformer path; multi-GPU sharding is a design note only.", file=sys.stderr)
        return 0

    if args.probe_traffic:
        return probe_traffic(args.n)
    if args.probe_contract:
        return probe_contract()
    if args.stack_only:
        print(json.dumps(stack_bench()), flush=True)
        return 0

    import torch
    from tt_boltz_amd import ops, pairformer, synthetic

    N, seed = args.n, 0
    dev = pairformer.get_device()
    w = synthetic.stack_weights(1, seed)
    s_cpu, z_cpu, _, _ = synthetic.pair_inputs(N, seed)
    pf = pairformer.Pairformer(1, 32, 4, 24, 16, True, w)
    layer = pf.blocks[0]
    ws = ops.workspace(pf.workspace_bytes(1, N), dev)
    z = z_cpu.to(dev).contiguous()
    s = s_cpu.to(dev).contiguous()
    stream = torch.cuda.current_stream()
    # layers run back to back as in a stack: each layer's single-track update runs on a
    # second stream, overlapped with the next layer's pair operations (Pairformer's
    # default schedule); the timed region ends after the last one has finished
    single = pf.single_track(1, N, dev)

    def step():
        layer(s, z, None, None, ws, 0, single)

    for _ in range(args.warmup):
        step()
    single.join()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_wall0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    single.join()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall0
    ms_step = e0.elapsed_time(e1) / args.steps
    if not torch.isfinite(z).all():
        print("non-finite z after timed steps", file=sys.stderr)
        return 1
    # the same layer with everything on one stream in reference order
    serial_ms = time_events(lambda: layer(s, z, None, None, ws), args.steps, stream)

    # per-op breakdown (each op timed alone, same stream, in-place like the layer)
    fl = flops_layer(N)

    def time_op(fn, reps=10):
        return time_events(fn, reps, stream)

    ops_ms = {
        "trimul_out": time_op(lambda: layer.triangle_multiplication_start(z, None, out=z, accumulate=True, ws=ws)),
        "trimul_in": time_op(lambda: layer.triangle_multiplication_end(z, None, out=z, accumulate=True, ws=ws)),
        "triatt_start": time_op(lambda: layer.triangle_attention_start(z, None, out=z, accumulate=True, ws=ws)),
        "triatt_end": time_op(lambda: layer.triangle_attention_end(z, None, out=z, accumulate=True, ws=ws)),
        "transition_z": time_op(lambda: layer.transition_z(z, out=z, accumulate=True, ws=ws)),
    }
    breakdown = {k: {"ms": round(v, 4)} for k, v in ops_ms.items()}
    for k, key in (("trimul_out", "trimul"), ("trimul_in", "trimul"), ("triatt_start", "triatt"),
                   ("triatt_end", "triatt"), ("transition_z", "transition_z")):
        breakdown[k]["tflops"] = round(fl[key] / (ops_ms[k] * 1e-3) / 1e12, 1)

    traffic = load_traffic()

    def counters_for(kname):
        """The committed PMC summary's entry for `kname` at this N (or None)."""
        if not traffic or traffic.get("N") != N:
            return None
        return traffic.get("kernels", {}).get(kname)

    def measured_traffic(kname):
        """Calibrated HBM bytes per launch of `kname` from the committed PMC summary (or None)."""
        k = counters_for(kname)
        return None if k is None else k["hbm_bytes_per_launch"]

    # Dominant kernel: the triangle-attention core (ta_attn_kernel, ~0.18 ms of each
    # triangle attention), launched alone on the q/k/v/bias/mask the last call left in the
    # workspace, timed with HIP events on the stream it runs on.  MFMA-bound: 4*N^3*128 FLOP
    # per launch (QK^T and PV over 4 heads of 32) against the traffic of q, k, v (16-bit) read
    # once, the fp32 bias of the 4 heads and the 16-bit mask once and o (16-bit) written once.
    # Its launch time is taken inside the layer loop: K more steps of the timed loop's schedule
    # (single track overlapped on the second stream) with every attention-core launch bracketed
    # by HIP events on the pair stream; the same kernel launched back to back on the operands
    # one call left in the workspace is reported beside it (warm caches, no neighbours).
    ops.attend_timing(True, layer.variant)
    for _ in range(args.steps):
        step()
    single.join()
    att_total_ms, att_launches = ops.attend_timing_read(layer.variant)
    ops.attend_timing(False, layer.variant)
    attn_ms = att_total_ms / max(att_launches, 1)
    reps = 20
    layer.triangle_attention_start(z, None, out=torch.empty_like(z), accumulate=False, ws=ws)
    iso_ms = time_op(lambda: ops.launch_triatt_attend(ws, 1, N, 0, layer.variant), reps)
    attn_flop = fl["triatt_core"]
    attn_tf = attn_flop / (attn_ms * 1e-3) / 1e12
    iso_tf = attn_flop / (iso_ms * 1e-3) / 1e12
    attn_bytes = (3 * 128 + 1 + 128) * N * N * 2 + 4 * N * N * 4
    mfma_live = ops.mfma_rate_probe(dev, variant=layer.variant)
    simds = 4 * torch.cuda.get_device_properties(dev).multi_processor_count
    roofline = {"kernel": "ta_attn_kernel", "bound": "mfma", "achieved": round(attn_tf, 1),
                "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(attn_tf / MFMA_BF16_PEAK_TFLOPS, 4),
                "traffic": measured_traffic("ta_attn_kernel"), "algorithmic_bytes": attn_bytes,
                "flop_per_launch": attn_flop, "exp_per_launch": N ** 3 * 4, "launch_ms": round(attn_ms, 4),
                "launch_ms_source": f"in-layer: mean of {att_launches} attention-core launches inside "
                                    f"{args.steps} layer steps (HIP events on the pair stream)",
                "isolated": {"launch_ms": round(iso_ms, 4), "achieved": round(iso_tf, 1),
                             "frac": round(iso_tf / MFMA_BF16_PEAK_TFLOPS, 4),
                             "note": f"{reps} back-to-back launches on one call's operands"},
                "hbm_gbs_algorithmic": round(attn_bytes / (attn_ms * 1e-3) / 1e9, 1),
                "measured_peak": {**mfma_live, "frac": round(attn_tf / mfma_live["tflops"], 4),
                                  "note": "sustained 16-bit MFMA rate of this chip under load (mfma_rate_kernel, "
                                          "random operands); achieved / this = frac of the loaded-clock peak"},
                "valu": valu_roof("ta_attn_kernel", N, attn_ms, simds, counters_for)}

    # The trimul contraction (the batched matmul of the triangle multiplication), launched
    # alone on its real operand planes (those the last trimul call left behind).  Below the
    # ridge point (2.5 PF / 8 TB/s = 312 FLOP/B) its 16-bit traffic binds: at N = 512 the
    # intensity is 171 FLOP/B.
    nplanes = 128
    plane_elems = nplanes * N * N
    dt = ops.TORCH_DTYPE[layer.variant]
    opA = ws[: plane_elems * 2].view(dt).view(nplanes, N, N)
    opB = ws[plane_elems * 2: plane_elems * 4].view(dt).view(nplanes, N, N)
    X = ws[plane_elems * 4: plane_elems * 6].view(dt).view(nplanes, N, N)
    layer.triangle_multiplication_start(z, None, out=torch.empty_like(z), accumulate=False, ws=ws)
    contract_ms = time_op(lambda: ops.launch_trimul_contract(opA, opB, X, layer.variant), reps)
    contract_flop = fl["trimul_contract"]       # 2*N^3*128: 128 planes of 2*N^3, one direction per launch
    achieved = contract_flop / (contract_ms * 1e-3) / 1e12
    kname = "tm_contract_dma_kernel" if N >= 384 else "tm_contract_kernel"
    alg_bytes = 3 * 128 * N * N * 2
    gbs = alg_bytes / (contract_ms * 1e-3) / 1e9
    mfma_part = {"achieved": round(achieved, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                 "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4)}
    bound_hbm = alg_bytes / (HBM_PEAK_GBS * 1e9) >= contract_flop / (MFMA_BF16_PEAK_TFLOPS * 1e12)
    contract = {"kernel": kname, "bound": "hbm" if bound_hbm else "mfma",
                **({"achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(gbs / HBM_PEAK_GBS, 4)} if bound_hbm else mfma_part),
                "traffic": measured_traffic(kname), "algorithmic_bytes": alg_bytes, "flop_per_launch": contract_flop,
                "intensity_flop_per_byte": round(contract_flop / alg_bytes, 1), "launch_ms": round(contract_ms, 4),
                "mfma": mfma_part}
    if traffic and traffic.get("N") == N:
        roofline["traffic_note"] = contract["traffic_note"] = traffic.get("note")

    # the same layer with bf16 MFMA operands (libpairformer_hip_bf16.so, same kernels)
    pf_bf16 = pairformer.Pairformer(1, 32, 4, 24, 16, True, w, pairformer.Options(operand="bf16"))
    zb, sb = z_cpu.to(dev).contiguous(), s_cpu.to(dev).contiguous()
    single_bf16 = pf_bf16.single_track(1, N, dev)

    def step_bf16():
        pf_bf16.blocks[0](sb, zb, None, None, ws, 0, single_bf16)

    # the schedule of the timed loop: the single track of step k beside the pair operations of
    # step k + 1, joined once after the last step
    for _ in range(args.warmup):
        step_bf16()
    single_bf16.join()
    torch.cuda.synchronize()
    be0, be1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    be0.record(stream)
    for _ in range(args.steps):
        step_bf16()
    single_bf16.join()
    be1.record(stream)
    torch.cuda.synchronize()
    bf16_ms = be0.elapsed_time(be1) / args.steps
    del pf_bf16, single_bf16

    # the same layer without the weight-precision paths (plain 16-bit weights: no hi + lo
    # residuals, no mean correction), for the cost of those paths
    pf_plain = pairformer.Pairformer(1, 32, 4, 24, 16, True, w,
                                     pairformer.Options(weight_residuals=False, mean_correction=False))
    zp, sp = z_cpu.to(dev).contiguous(), s_cpu.to(dev).contiguous()
    single_plain = pf_plain.single_track(1, N, dev)

    def step_plain():
        pf_plain.blocks[0](sp, zp, None, None, ws, 0, single_plain)

    for _ in range(args.warmup):
        step_plain()
    single_plain.join()
    torch.cuda.synchronize()
    pe0, pe1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    pe0.record(stream)
    for _ in range(args.steps):
        step_plain()
    single_plain.join()
    pe1.record(stream)
    torch.cuda.synchronize()
    plain_ms = pe0.elapsed_time(pe1) / args.steps
    # the cost of the precision paths from interleaved rounds (precision layer, then plain layer,
    # K steps each, three times), so that clock drift between two separately timed loops does
    # not enter the ratio; `value` stays the main timed loop above
    def time_steps(stepf, single_track):
        a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a0.record(stream)
        for _ in range(args.steps):
            stepf()
        single_track.join()
        a1.record(stream)
        torch.cuda.synchronize()
        return a0.elapsed_time(a1) / args.steps
    inter = [(time_steps(step, single), time_steps(step_plain, single_plain)) for _ in range(3)]
    inter_ratio = sorted(p / q for p, q in inter)[1]
    del pf_plain, single_plain, zp, sp

    # the same layer on padded inputs as a caller passes them: the last 51 of the N tokens are
    # padding (token and pair masks, n_valid), the schedule as in the timed loop
    pad_tail = 51
    _, z_pad, mask_pad, pm_pad = synthetic.pair_inputs(N, seed, pad_tail=pad_tail, with_s=False)
    zq, sq = z_pad.to(dev).contiguous(), s_cpu.to(dev).contiguous()
    mq, pmq = mask_pad.to(dev).contiguous(), pm_pad.to(dev).contiguous()
    single_pad = pf.single_track(1, N, dev)

    def step_pad():
        layer(sq, zq, pmq, mq, ws, N - pad_tail, single_pad)

    for _ in range(args.warmup):
        step_pad()
    single_pad.join()
    torch.cuda.synchronize()
    qe0, qe1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    qe0.record(stream)
    for _ in range(args.steps):
        step_pad()
    single_pad.join()
    qe1.record(stream)
    torch.cuda.synchronize()
    pad_ms = qe0.elapsed_time(qe1) / args.steps
    del single_pad, zq, sq, mq, pmq

    out = {
        "metric": "Pairformer layers/sec at N=512, fp16 MFMA operands (bf16-operand rate in operand_variants)",
        "value": round(1000.0 / ms_step, 3),
        "unit": "layers/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "operand_variants": {"fp16_layers_per_s": round(1000.0 / ms_step, 3),
                             "bf16_layers_per_s": round(1000.0 / bf16_ms, 3),
                             "note": "MFMA operand type (fp32 accumulate, fp32 residual stream). BASELINE names "
                                     "bf16; value is the fp16-operand layer (same 16-bit MFMA rate, 3 more "
                                     "mantissa bits), the default because bf16 operands miss the 2e-3 "
                                     "mean-error bar; bf16_layers_per_s is the bf16-operand build"},
        "single_stream_layers_per_s": round(1000.0 / serial_ms, 3),
        "padded_input": {"layers_per_s": round(1000.0 / pad_ms, 3), "ms_per_step": round(pad_ms, 4),
                         "n_valid": N - pad_tail,
                         "note": f"the same layer with the last {pad_tail} of {N} tokens padded (token and pair "
                                 "masks given, n_valid set), as a caller's padded batch arrives"},
        "precision_paths": {"plain16_layers_per_s": round(1000.0 / plain_ms, 3),
                            "cost_pct": round(100.0 * (inter_ratio - 1.0), 2),
                            "cost_pct_separate": round(100.0 * (ms_step / plain_ms - 1.0), 2),
                            "interleaved_ms": [[round(p, 4), round(q, 4)] for p, q in inter],
                            "note": "value runs the weight-precision paths (hi + lo weights in the trimul "
                                    "output, triangle-attention gate/output and recycling projections; the "
                                    "mean correction of the trimul's and triangle attention's input "
                                    "projections and of the pair transition's fc3); plain16 is the same "
                                    "layer with every weight a single 16-bit rounding. cost_pct: median "
                                    "ratio of three interleaved rounds (precision, plain; ms per layer in "
                                    "interleaved_ms); cost_pct_separate: value against the plain loop "
                                    "timed once on its own"},
        "data": "synthetic (seeded N(0,1) inputs, random-init weights, seed 0)",
        "config": {"workload": f"one Boltz-2 PairformerLayer, N={N}, c_z=128, c_s=384, tri-att 4x32, "
                               f"single-att 16x24, masks all ones, device-resident fp32 z/s; layers back to "
                               f"back as in a stack (single track overlapped with the next layer's pair ops "
                               f"on a second stream)",
                   "N": N, "batch": 1, "layer_tflop": round(fl["layer"] / 1e12, 4),
                   "layer_tflops_achieved": round(fl["layer"] / (ms_step * 1e-3) / 1e12, 1)},
        "roofline": roofline,
        "roofline_contract": contract,
        "breakdown": breakdown,
        "wall_s_timed": round(wall, 3),
        "device": torch.cuda.get_device_name(0),
        "host": platform.node(),
    }
    if not args.no_stack:
        del zb, sb
        out["contract_vs_hipblaslt"] = contract_vs_library()
        torch.cuda.empty_cache()
        out["stack"] = stack_bench()
        torch.cuda.empty_cache()
        out["fast"] = fast_bench()
        torch.cuda.empty_cache()
        out["fast_trunk"] = fast_trunk_bench()
        torch.cuda.empty_cache()
        out["msa"] = msa_bench()
        torch.cuda.empty_cache()
        out["diffusion_pair"] = diffusion_bench()
        torch.cuda.empty_cache()
        out["template"] = template_bench()
        torch.cuda.empty_cache()
        out["msa_trunk"] = msa_trunk_bench()
        torch.cuda.empty_cache()
        out["module_end_to_end"] = module_bench()
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(N, seed)
        if "stack" in out:
            # config 3 on the CPU: one layer at N=768 timed once, extrapolated to 64 layers x 4 passes
            c3 = cpu_baseline(out["stack"]["N"], 3, reps=1)
            layer_s = 1.0 / c3["value"]
            out["stack"]["cpu_extrapolated"] = {
                "trunk_s": round(layer_s * out["stack"]["layers"] * out["stack"]["passes"], 1),
                "layer_s": round(layer_s, 2), "cores": c3["cores"], "kind": "port",
                "note": "extrapolated: 1 PairformerLayer at N=768 on the fp32 CPU oracle, x64 layers x4 passes"}
            out["cpu_configs"] = cpu_configs()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
