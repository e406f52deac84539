"""`python -m gpt_from_scratch_amd.harness --steps 10 --warmup 3`: the config-5
train step alone (gpt.py), its timed steps inside profiler regions."""
import argparse
import json

from ..profiler_regions import ProfilerRegions
from .gpt import GPTConfig, train

ap = argparse.ArgumentParser(description="config-5 GPT train step on the HIP kernels")
ap.add_argument("--steps", type=int, default=10)
ap.add_argument("--warmup", type=int, default=3)
args = ap.parse_args()
losses, tps = train(GPTConfig(), 8, 1024, steps=args.steps, seed=5, device="cuda",
                    warmup=args.warmup, regions=ProfilerRegions())
print(json.dumps({"tokens_per_s": round(tps, 1), "ms_per_step": round(8 * 1024 / tps * 1e3, 3),
                  "steps": args.steps, "warmup": args.warmup, "loss_last": round(losses[-1], 4)}),
      flush=True)
