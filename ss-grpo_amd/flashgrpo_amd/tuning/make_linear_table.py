"""Regenerate the projection-path table (run on the MI355X it is meant for).

    python -m flashgrpo_amd.tuning.make_linear_table --out linear_mi355x.csv
        [--presets qwen25_1p5b,...] [--rows 416,...] [--kinds qkv,o,down] [--plan TM,TN,S,NS] [--reps 10]

For the QKV, O and down projections of every bf16 target preset and a grid of row counts
(powers of two plus the verify-round shapes of the benchmark workloads), it times the two ways
a decoder layer can compute the projection together with the op that consumes it:

* the library GEMM (hipBLASLt through the GEMM solution table) followed by ``fg_rope_kv_write``
  (QKV, with its bias in the GEMM) or added into the residual stream (``addmm_``) and followed
  by ``fg_rmsnorm`` (O, down);
* ``fg_linear_parts`` followed by the kernel that finishes its fp32 parts
  (``fg_rope_kv_write_parts``, ``fg_residual_rmsnorm_parts``), over tile sizes and split counts
  that put between 64 and 1024 workgroups on the chip, with a 2- or 4-stage LDS ring;
* for QKV also ``fg_linear_rope_kv_write`` (one split, the bias, rotary embedding and cache write
  in the GEMM's epilogue) over the tile sizes and rings, written as kind ``qkv_rope`` with the
  same library time and the fused time in the split-K columns.

The verify forward replays its launches as a HIP graph, so each path is timed the same way: one
graph holding ``batch`` back-to-back calls, the weight rotating over enough copies to exceed the
256 MB last-level cache (so it is read from HBM, as in a forward over all layers), replayed
``reps`` times between events; a call's time is the fastest replay divided by ``batch``. (Events
around single eager launches add the launch gaps, which would favour whichever path has the
shorter kernels at small shapes.) One row per shape names the faster path and the best split-K
tile and split count. ``--presets`` / ``--rows`` / ``--kinds`` restrict the run and ``--plan`` times
one split-K plan instead of the sweep (a profiling run of one shape); the full table needs none.
"""
from __future__ import annotations

import argparse
import os
import sys

GRID = (64, 128, 256, 512, 1024, 2048)
# preset -> verify-round row counts (sequences x tree nodes) of the benchmark workloads
SHAPES = {
    "qwen25_1p5b": (32 * 13,),
    "qwen25_7b": (64 * 13, 64 * 29),
    "qwen25_14b": (128 * 41,),
    "llama31_8b": (96 * 48,),
}
TILES = ((64, 64), (64, 128), (128, 64), (128, 128))
STAGES = (2, 4)


def split_candidates(K, rows, cols, hidden):
    """(tile_m, tile_n, splits, stages) with 64-1024 workgroups (one split when the tiles alone
    exceed that), at least two k-steps per split, and a 2- or 4-stage ring."""
    out = []
    nk = hidden // 64
    for tm, tn in TILES:
        tiles = -(-rows // tm) * -(-cols // tn)
        if tiles >= 1024:
            out += [(tm, tn, 1, ns) for ns in STAGES]
            continue
        for s in range(1, nk // 2 + 1):
            if K.linear_splits(hidden, s) == s and 64 <= tiles * s <= 1024:
                out += [(tm, tn, s, ns) for ns in STAGES]
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--out", required=True)
    ap.add_argument("--reps", type=int, default=10)
    ap.add_argument("--presets", default="", help="comma-separated preset names (default: all)")
    ap.add_argument("--rows", default="", help="comma-separated row counts (default: the full grid)")
    ap.add_argument("--kinds", default="", help="comma-separated projections: qkv, o, down (default: all)")
    ap.add_argument("--plan", default="", help="tile_m,tile_n,splits,stages: time this split-K plan only")
    args = ap.parse_args()
    only_kinds = {k for k in args.kinds.split(",") if k}
    plan = tuple(int(v) for v in args.plan.split(",")) if args.plan else None
    only_presets = {p for p in args.presets.split(",") if p}
    only_rows = {int(r) for r in args.rows.split(",") if r}
    import torch
    import torch.nn.functional as F

    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
    from flashgrpo_amd import kernels as K
    from flashgrpo_amd.models.target import TargetConfig, inv_freq_table
    from flashgrpo_amd.tuning import use_tuned_gemms

    use_tuned_gemms()
    dev = "cuda"

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

    lines = ["kind,rows,cols,hidden,library_us,split_k_us,tile_m,tile_n,splits,stages,choice"]
    for preset, extra in SHAPES.items():
        if only_presets and preset not in only_presets:
            continue
        cfg = getattr(TargetConfig, preset)()
        H, d, Hq, Hkv = cfg.hidden, cfg.head_dim, cfg.q_heads, cfg.kv_heads
        inv = inv_freq_table(d, cfg.rope_theta).to(dev)
        kinds = (("qkv", (Hq + 2 * Hkv) * d, H), ("o", H, Hq * d), ("down", H, cfg.intermediate))
        for kind, N, Kd in kinds:
            if only_kinds and kind not in only_kinds:
                continue
            g = torch.Generator(device=dev).manual_seed(N + Kd)
            copies = min(32, max(2, -(-512 * 2 ** 20 // (N * Kd * 2))))
            batch = max(copies, 8)
            ws = [(torch.randn(N, Kd, device=dev, generator=g) * 0.02).to(torch.bfloat16) for _ in range(copies)]
            bias = (torch.randn(N, device=dev, generator=g) * 0.02).to(torch.bfloat16) if cfg.qkv_bias else None
            norm_w = torch.ones(H, dtype=torch.bfloat16, device=dev)
            wp = bp = None  # pair-interleaved copies for the fused QKV epilogue, made on first use
            for rows in sorted(only_rows or (set(GRID) | set(extra))):
                x = (torch.randn(rows, Kd, device=dev, generator=g) * 0.5).to(torch.bfloat16)
                res = torch.randn(rows, H, device=dev, generator=g).to(torch.bfloat16)
                h = torch.empty(rows, H, dtype=torch.bfloat16, device=dev)
                it = [0]

                def w_next():
                    it[0] += 1
                    return ws[it[0] % copies]

                if kind == "qkv":
                    nodes = next(n for n in (13, 29, 41, 48, 16, 8, 4, 2, 1) if rows % n == 0)
                    B = rows // nodes
                    kc = torch.zeros(B, Hkv, 64, d, dtype=torch.bfloat16, device=dev)
                    vc = torch.zeros_like(kc)
                    q = torch.empty(B, nodes, Hq, d, dtype=torch.bfloat16, device=dev)
                    sl = torch.zeros(B, dtype=torch.int32, device=dev)
                    po = torch.arange(nodes, dtype=torch.int32, device=dev)
                    rope = dict(batch=B, num_nodes=nodes, q_heads=Hq, kv_heads=Hkv, head_dim=d, seq_len=sl,
                                pos_offset=po, inv_freq=inv, q_out=q, k_cache=kc, v_cache=vc)

                    def library():
                        K.rope_kv_write(F.linear(x, w_next(), bias), **rope)

                    def split_k(tm, tn, s, ns, buf):
                        def run():
                            K.rope_kv_write_parts(K.linear_parts(x, w_next(), splits=s, tile=(tm, tn), stages=ns,
                                                                 out=buf), bias, **rope)
                        return run
                else:
                    def library():
                        res.addmm_(x, w_next().t())
                        K.rmsnorm(res, norm_w, cfg.rms_eps, out=h)

                    def split_k(tm, tn, s, ns, buf):
                        def run():
                            K.residual_rmsnorm_parts(K.linear_parts(x, w_next(), splits=s, tile=(tm, tn), stages=ns,
                                                                    out=buf), res, norm_w, cfg.rms_eps, out=h)
                        return run

                t_lib = best(library, batch)
                top = None
                for tm, tn, s, ns in ([plan] if plan else split_candidates(K, rows, N, Kd)):
                    buf = torch.empty(s, rows, N, dtype=torch.float32, device=dev)
                    t = best(split_k(tm, tn, s, ns, buf), batch)
                    del buf
                    if top is None or t < top[0]:
                        top = (t, tm, tn, s, ns)
                choice = "split_k" if top[0] < t_lib else "library"
                lines.append(f"{kind},{rows},{N},{Kd},{t_lib:.1f},{top[0]:.1f},{top[1]},{top[2]},{top[3]},{top[4]},"
                             f"{choice}")
                print(f"{cfg.name} {kind} rows {rows}: library {t_lib:.1f}, split-K {top[0]:.1f} "
                      f"(tile {top[1]}x{top[2]}, {top[3]} splits, {top[4]} stages) -> {choice}", flush=True)
                if kind == "qkv" and not plan:
                    if wp is None:
                        wp = [K.rope_pair_rows(w, Hq, Hkv, d) for w in ws]
                        bp = None if bias is None else K.rope_pair_rows(bias, Hq, Hkv, d)
                    # the rows' rotary table: made once per forward for all layers, so outside the timing
                    cs = K.rope_cos_sin(batch=B, num_nodes=nodes, head_dim=d, seq_len=sl, pos_offset=po, inv_freq=inv)
                    fused_rope = {k: v for k, v in rope.items() if k not in ("pos_offset", "inv_freq")}
                    fused = None
                    for tm, tn in TILES:
                        for ns in STAGES:
                            def run(tm=tm, tn=tn, ns=ns):
                                it[0] += 1
                                K.linear_rope_kv_write(x, wp[it[0] % copies], bp, tile=(tm, tn), stages=ns,
                                                       cos_sin=cs, **fused_rope)
                            t = best(run, batch)
                            if fused is None or t < fused[0]:
                                fused = (t, tm, tn, ns)
                    choice = "split_k" if fused[0] < t_lib else "library"
                    lines.append(f"qkv_rope,{rows},{N},{Kd},{t_lib:.1f},{fused[0]:.1f},{fused[1]},{fused[2]},1,"
                                 f"{fused[3]},{choice}")
                    print(f"{cfg.name} qkv_rope rows {rows}: library {t_lib:.1f}, fused {fused[0]:.1f} "
                          f"(tile {fused[1]}x{fused[2]}, {fused[3]} stages)", flush=True)
                del x, res, h
            del ws
            torch.cuda.empty_cache()
    with open(args.out, "w") as f:
        f.write("\n".join(lines) + "\n")


if __name__ == "__main__":
    main()
