"""Writes minicpm2b_b16_chains.npz: the CPU oracle's greedy chains for the
batch-16 decoder test at the MiniCPM-2B shape (seed-3
weights, 16 prompts of 128 ids from make_prompts(seed=3), 64 greedy steps).

tokens [16][65] int32 (the prefill's argmax, then 64 decode steps) and
margins [16][65] float32 (top-1 minus top-2 logit of each step), from
oracle.DecoderOracle.generate. The oracle is deterministic and independent
of its thread count, so the chains equal a run on any host.

    python tests/golden/make_decoder_chains.py
"""
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle  # noqa: E402
from sparrow_amd import model as M  # noqa: E402

OUT = Path(__file__).resolve().parent / "minicpm2b_b16_chains.npz"
BATCH, PROMPT, STEPS = 16, 128, 64


def main():
    cfg = M.minicpm_2b_config()
    W = M.make_weights(cfg, seed=3)
    prompts = M.make_prompts(cfg, BATCH, PROMPT, seed=3)
    toks = np.empty((BATCH, STEPS + 1), np.int32)
    margins = np.empty((BATCH, STEPS + 1), np.float32)
    for b in range(BATCH):
        t = time.time()
        ref = oracle.DecoderOracle(W, cfg, cap=PROMPT + STEPS + 8)
        toks[b], margins[b] = ref.generate(prompts[b], STEPS)
        print(f"sequence {b}: {time.time() - t:.1f}s, min margin {margins[b].min():.3e}",
              flush=True)
    np.savez(OUT, tokens=toks, margins=margins, prompts=prompts)
    print(OUT)


if __name__ == "__main__":
    main()
