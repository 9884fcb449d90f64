"""Which operand rounding drives the stack-depth drift (config 3).

Runs the 64-layer N = 768 trunk with 3 recycling steps (seed 3, as in
``test_gpu_stack.test_config3_stack_depth``) through the fp32 oracle on the device, once
exactly and once per operand selector of ``pairformer_ref.operand_rounding`` (one family of
rounding sites rounded to fp16 at a time), and prints each selector's drift from the exact
run after every pass, as mean |d| / rms and max |d| / rms of z and s.  Optional: the GPU
stack itself (``--gpu``) under the same statistics.

    python tests/precision_ablation.py [--n 768] [--blocks 64] [--steps 3] [--gpu]
        [--select tm_ab ta_p ...] [--json out.json]

A selector is a family name, a site (``ta_qk.x``), ``x`` / ``w`` (that side of every family),
an exclusion ``!<item>``, ``all``, or several joined with ``+``; a ``~meanfix`` suffix applies
each rounded weight's error to the activation's deviation from its mean over positions only
(``~meanfix=<selector>``: at those weight sites only; ``@k``: the mean over every k-th position);
``build`` is this build's precision model (``pairformer_ref.BUILD_MODEL``).  Not collected by pytest (test infrastructure that
needs a GPU and minutes).
"""
import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from oracle import pairformer_ref as ref  # noqa: E402
from tt_boltz_amd import synthetic  # noqa: E402

DEFAULT = ["all", "w", "x"] + list(f for f in ref.FAMILIES if f != "misc")


def stats(got, want):
    d = (got.double() - want.double()).abs()
    rms = want.double().pow(2).mean().sqrt()
    return (d.max() / rms).item(), (d.mean() / rms).item()


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--n", type=int, default=768)
    ap.add_argument("--blocks", type=int, default=64)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--gpu", action="store_true", help="also the GPU stack (this build's kernels)")
    ap.add_argument("--select", nargs="*", default=DEFAULT)
    ap.add_argument("--gpu-variants", nargs="*", default=["gpu"],
                    choices=["gpu", "gpu-no-meanfix", "gpu-plain"],
                    help="with --gpu: the full build, without the mean correction, without any residual")
    ap.add_argument("--json", default=None)
    args = ap.parse_args(argv)
    dev = torch.device("cuda", 0) if torch.cuda.is_available() else torch.device("cpu")
    cfg = synthetic.CONFIGS[3]
    N, n_blocks, steps = args.n, args.blocks, args.steps
    w = synthetic.stack_weights(n_blocks, cfg["seed"])
    w_rec = synthetic.draw(synthetic.recycle_shapes(), cfg["seed"] + 1000)
    s_init, z_init, mask, _ = synthetic.pair_inputs(N, cfg["seed"], z_scale=cfg["z_scale"])
    wd = {k: v.to(dev) for k, v in w.items()}
    wrd = {k: v.to(dev) for k, v in w_rec.items()}
    sd, zd, md = s_init.to(dev), z_init.to(dev), mask.to(dev)

    def run(select):
        out = []
        if select.split("@")[0] == "build":   # this build's precision model (optionally @k sampled means)
            t0 = time.time()
            k = int(select.split("@")[1]) if "@" in select else 1
            with torch.no_grad(), ref.operand_rounding(torch.float16, **ref.BUILD_MODEL, mean_sample=k):
                ref.recycle(sd, zd, md, wd, wrd, n_blocks, steps,
                            pass_hook=lambda i, s, z: out.append((s.clone(), z.clone())))
            return out, time.time() - t0
        sel, _, fix = select.partition("~")
        mean_fix, sample = False, 1
        if fix:   # "meanfix", "meanfix=<selector>", optionally "@<k>" (every k-th position)
            fix, _, k = fix.partition("@")
            sample = int(k) if k else 1
            name, _, fsel = fix.partition("=")
            assert name == "meanfix", select
            mean_fix = fsel.split("+") if fsel else True
        fams = None if sel in ("all", "exact") else sel.split("+")
        t0 = time.time()
        with torch.no_grad(), ref.operand_rounding(None if sel == "exact" else torch.float16, fams, mean_fix,
                                                   sample):
            ref.recycle(sd, zd, md, wd, wrd, n_blocks, steps,
                        pass_hook=lambda i, s, z: out.append((s.clone(), z.clone())))
        if dev.type == "cuda":
            torch.cuda.synchronize()
        return out, time.time() - t0

    exact, dt = run("exact")
    print(f"[ablation] exact oracle: {dt:.1f} s", flush=True)
    rows = {}

    def report(name, got):
        per = []
        for i in range(steps + 1):
            zmx, zmn = stats(got[i][1], exact[i][1])
            smx, smn = stats(got[i][0], exact[i][0])
            per.append({"z_max": zmx, "z_mean": zmn, "s_max": smx, "s_mean": smn})
        rows[name] = per
        cells = " | ".join(f"p{i} z {p['z_mean']:.2e}/{p['z_max']:.2e} s {p['s_mean']:.2e}"
                           for i, p in enumerate(per))
        print(f"[ablation] {name:>14}: {cells}", flush=True)

    for sel in args.select:
        got, dt = run(sel)
        report(sel, got)
        del got
    if args.gpu:
        from tt_boltz_amd import pairformer
        variants = {"gpu": {}, "gpu-no-meanfix": {"mean_correction": False},
                    "gpu-plain": {"mean_correction": False, "weight_residuals": False}}
        for name in args.gpu_variants:
            pf = pairformer.Pairformer(n_blocks, 32, 4, 24, 16, True, w, pairformer.Options(**variants[name]))
            rec = pairformer.TrunkRecycler(pf, w_rec)
            got = []
            rec(sd.contiguous(), zd.contiguous(), md, steps,
                pass_hook=lambda i, s, z: got.append((s.clone(), z.clone())))
            if dev.type == "cuda":
                torch.cuda.synchronize()
            report(name, got)
            del pf, rec, got
    if args.json:
        with open(args.json, "w") as f:
            json.dump({"N": N, "blocks": n_blocks, "steps": steps, "rows": rows}, f, indent=1)


if __name__ == "__main__":
    main()
