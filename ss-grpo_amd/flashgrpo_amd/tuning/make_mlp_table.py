"""Regenerate the MLP input-path table (run on the MI355X it is meant for).

    python -m flashgrpo_amd.tuning.make_mlp_table --out mlp_mi355x.csv [--reps 10]
        [--presets qwen25_7b,...] [--rows 1856,...]

For the (intermediate, hidden) sizes of every target preset and a grid of row counts
(powers of two plus the verify-round and prefill shapes of the benchmark workloads), it
times the two ways the decoder layer can compute its MLP input SiLU(x.Wg^T) * (x.Wu^T):
the hipBLASLt projection (through the GEMM solution table) followed by ``fg_swiglu``, and
``fg_gate_up_swiglu`` at each tile height (64, 128, 192, 256 rows). The verify forward replays
its launches as a HIP graph, so each path is timed as one graph of ``batch`` back-to-back calls
with the weight rotating over enough copies to exceed the 256 MB last-level cache (so it is read
from HBM), replayed ``reps`` times; a call's time is the fastest replay divided by ``batch``.
One row per shape names the fastest path. ``--presets`` / ``--rows`` restrict the run to some
presets and row counts (a profiling run of one shape); the full table needs neither.
"""
from __future__ import annotations

import argparse
import os
import sys

GRID = (64, 128, 256, 512, 1024, 2048, 4096, 8192)
TILES = (64, 128, 192, 256)
# preset -> extra row counts: verify rounds (sequences x tree nodes) and prefill chunks
# (prompts x chunk) of the benchmark workloads
SHAPES = {
    "tiny": (8 * 16, 4 * 256),
    "qwen25_1p5b": (32 * 13, 32 * 16, 4 * 512),
    "qwen25_7b": (64 * 13, 64 * 29, 64 * 32),
    "qwen25_14b": (128 * 41, 16 * 1024),
    "llama31_8b": (96 * 48, 12 * 1024),
}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--out", required=True)
    ap.add_argument("--reps", type=int, default=10)
    ap.add_argument("--presets", default="", help="comma-separated preset names (default: all)")
    ap.add_argument("--rows", default="", help="comma-separated row counts (default: the full grid)")
    args = ap.parse_args()
    only_presets = {p for p in args.presets.split(",") if p}
    only_rows = {int(r) for r in args.rows.split(",") if r}
    import torch
    import torch.nn.functional as F

    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
    from flashgrpo_amd import kernels as K
    from flashgrpo_amd.models.target import TargetConfig
    from flashgrpo_amd.tuning import use_tuned_gemms

    use_tuned_gemms()

    def best(fn, batch):
        fn()  # eager first: library handles, workspaces and the TunableOp lookup outside the graph
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(batch):
                fn()
        g.replay()
        ts = []
        for _ in range(args.reps):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            g.replay()
            e.record()
            e.synchronize()
            ts.append(s.elapsed_time(e) * 1e3 / batch)
        del g
        return min(ts)

    paths = ("pair",) + tuple(f"fused{t}" for t in TILES)
    lines = ["rows,inter,hidden," + ",".join(f"{k}_us" for k in paths) + ",choice"]
    done = set()
    for preset, extra in SHAPES.items():
        if only_presets and preset not in only_presets:
            continue
        cfg = getattr(TargetConfig, preset)()
        I, H = cfg.intermediate, cfg.hidden
        if (I, H) in done:
            continue
        done.add((I, H))
        g = torch.Generator(device="cuda").manual_seed(I)
        copies = min(16, max(2, -(-512 * 2 ** 20 // (2 * I * H * 2))))
        batch = max(copies, 8)
        ws = [(torch.randn(2 * I, H, device="cuda", generator=g) * 0.05).to(torch.bfloat16) for _ in range(copies)]
        for rows in sorted(only_rows or (set(GRID) | set(extra))):
            x = (torch.randn(rows, H, device="cuda", generator=g) * 0.5).to(torch.bfloat16)
            out = torch.empty(rows, I, dtype=torch.bfloat16, device="cuda")
            it = [0]

            def pair():
                it[0] += 1
                K.swiglu(F.linear(x, ws[it[0] % copies]), out=out)

            def fused(tile):
                def run():
                    it[0] += 1
                    K.gate_up_swiglu(x, ws[it[0] % copies], out=out, tile_rows=tile)
                return run

            t = {"pair": best(pair, batch)}
            for tile in TILES:
                t[f"fused{tile}"] = best(fused(tile), batch)
            choice = min(t, key=t.get)
            lines.append(f"{rows},{I},{H}," + ",".join(f"{t[k]:.1f}" for k in paths) + f",{choice}")
            print(f"{cfg.name} rows {rows}: " + ", ".join(f"{k} {v:.1f}" for k, v in t.items()) + f" -> {choice}",
                  flush=True)
            del x, out
        del ws
        torch.cuda.empty_cache()
    with open(args.out, "w") as f:
        f.write("\n".join(lines) + "\n")


if __name__ == "__main__":
    main()
