"""Regenerate gemm_gfx950.csv: run one C4-size aggregator forward under TunableOp tuning.

    python 4d_ttt_merging_amd/tuning/tune_gemms.py [--out PATH] [--frames 32]

Every distinct GEMM of the forward (qkv, output projection, MLP, at the frame,
register and merged global blocks' row counts) is benchmarked over the
hipBLASLt and rocBLAS solutions (up to 200 iterations or 200 ms each) and the
fastest is written to the table.  Needs an MI355X; takes about ten seconds.
"""
from __future__ import annotations

import argparse
import importlib
import sys
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[2]


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default=str(Path(__file__).with_name("gemm_gfx950.csv")))
    ap.add_argument("--frames", type=int, default=32)
    args = ap.parse_args()
    sys.path.insert(0, str(ROOT))
    agg = importlib.import_module("4d_ttt_merging_amd.aggregator")
    device = torch.device("cuda", 0)
    torch.manual_seed(0)
    model = agg.Aggregator(embed_dim=1024, depth=24, num_heads=16, num_register_tokens=4).to(device).eval()
    patches = torch.randn(args.frames, 32 * 32, 1024, device=device)
    model.set_input_patch_tokens_cache(patches)
    model.set_fastvggt(True, merge_ratio=0.5, protect_ratio=0.0, mass_bias=True)
    images = torch.zeros(1, args.frames, 3, 512, 512, device=device)
    tunable = torch.cuda.tunable
    tunable.enable(True)
    tunable.tuning_enable(True)
    tunable.set_filename(args.out)
    tunable.set_max_tuning_duration(200)
    tunable.set_max_tuning_iterations(200)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        model(images)
    torch.cuda.synchronize()
    tunable.tuning_enable(False)
    print(f"tuned {len(tunable.get_results())} GEMM shapes -> {args.out}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
