"""Regenerate the GEMM solution table (run on the MI355X it is meant for).

    python -m flashgrpo_amd.tuning.make_gemm_table --out gemm_mi355x.csv [--configs 7b,1.5b,14b,8b]

For each workload it builds the random-init target model and runs the verify
forward at the rollout shape (sequences x tree nodes) and the prefill chunk
shape with TunableOp tuning on, so exactly the GEMM calls of the forward are
tuned; TunableOp writes the table when the process exits.
"""
from __future__ import annotations

import argparse
import os
import sys

# (target preset, dtype, rollout rows = sequences x tree nodes, prefill rows = prompts x 64)
WORKLOADS = {
    "7b": ("qwen25_7b", 64 * 29, 8 * 64),
    "1.5b": ("qwen25_1p5b", 32 * 13, 4 * 64),
    "14b": ("qwen25_14b", 128 * 41, 16 * 64),
    "8b": ("llama31_8b", 96 * 48, 12 * 64),
}
SEQUENCES = {"7b": 64, "1.5b": 32, "14b": 128, "8b": 96}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--out", required=True)
    ap.add_argument("--configs", default="7b,1.5b,14b,8b")
    args = ap.parse_args()
    os.environ["FLASHGRPO_AMD_GEMM_TABLE"] = "off"
    import torch
    import torch.cuda.tunable as tunable

    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
    from flashgrpo_amd.models.target import TargetConfig, TargetModel, as_mask_tensor, chain_bits

    tunable.enable(True)
    tunable.tuning_enable(True)
    tunable.set_filename(os.path.abspath(args.out), insert_device_ordinal=False)
    for name in args.configs.split(","):
        preset, rollout_rows, prefill_rows = WORKLOADS[name]
        cfg = getattr(TargetConfig, preset)()
        model = TargetModel.random(cfg, seed=0, dtype=torch.bfloat16, device="cuda")
        for rows in (rollout_rows, prefill_rows):
            n = 64 if rows == prefill_rows else rows // SEQUENCES[name]
            b = rows // n
            cache = model.new_cache(b, 2 * n + 8)
            seq = torch.zeros(b, dtype=torch.int32, device="cuda")
            tok = torch.zeros((b, n), dtype=torch.int32, device="cuda")
            model.forward(tok, cache, pos_offset=torch.arange(n, dtype=torch.int32, device="cuda"),
                          anc=as_mask_tensor(chain_bits(n), "cuda"), seq_len=seq)
            torch.cuda.synchronize()
            print(f"tuned {name} rows {rows}", flush=True)
        del model, cache
        torch.cuda.empty_cache()


if __name__ == "__main__":
    main()
