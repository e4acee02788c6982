"""Write tests/golden/c5_greedy.json: the greedy ids of config 5 on the
reference's own kernels.

    make -C oracle && python tests/golden/make_c5_greedy.py [--threads N]

Config 5: the LLaMA-2-7B-architecture model with random
N(0, 0.02) weights quantized Q4_K_M (Q6_K for attn_v, ffn_down and the head;
llm_core_amd.model.SynthLlama(LLAMA2_7B, seed=5)), context 2048, a 512-token
prompt (BOS = 1 followed by 511 ids from numpy's PCG64 seed 5; the reference
prepends BOS only when the prompt does not start with it,
llama_model.cpp:1563-1566), then 32 greedy tokens with temperature 0, no
repetition penalty and no EOS stop.

The generation is llama_generate_cpu_impl's (llama_model.cpp:1502-1631) run by
ref_generate_greedy (oracle/ref_shim.cpp): one llama_forward_batch of the
prompt and one llama_forward_token per generated token on the reference's
x86 kernels compiled from their sources (the Q4_K GEMM and the r8 / 4-row
Q8_0 GEMVs, AVX-VNNI where the CPU has it, on the reference ThreadPool), with
the glue ops from the oracle's restatement.  tests/test_oracle_ref.py checks
that this generator gives the same ids and margins bit for bit as the
oracle's orc_generate_greedy on small models.

Stored: the prompt, the 32 ids, per id the top-1 minus top-2 margin of the
logits it was taken from (how close the reference's own choice was) and the
step's 8 largest logits with their ids, plus the model and prompt parameters.
Plain JSON.
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from llm_core_amd.model import LLAMA2_7B, Hparams, SynthLlama  # noqa: E402
from oracle import oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent / "c5_greedy.json"
N_PROMPT, N_GEN, N_CTX, SEED, TOP_K = 512, 32, 2048, 5, 8


def c5_prompt(n_vocab: int) -> np.ndarray:
    rest = np.random.default_rng(SEED).integers(0, n_vocab, N_PROMPT - 1)
    return np.concatenate([[1], rest]).astype(np.int32)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=0, help="reference ThreadPool size (0: min(16, nproc))")
    args = ap.parse_args()
    if O.ref is None:
        print("oracle/_ref not built (make -C oracle where the reference tree exists)", file=sys.stderr)
        return 1
    hp = Hparams(n_ctx=N_CTX, **LLAMA2_7B)
    t0 = time.time()
    model = SynthLlama(hp, seed=SEED)
    prompt = c5_prompt(hp.n_vocab)
    om = O.OracleModel(hp, model.tensors)
    print(f"model synthesised in {time.time() - t0:.0f} s; generating ...", file=sys.stderr, flush=True)
    t0 = time.time()
    ids, margins, top_ids, top_vals = O.ref_generate_greedy(om, prompt, N_GEN, args.threads, top_k=TOP_K)
    om.close()
    dt = time.time() - t0
    out = {
        "what": "config 5 greedy ids on the reference's x86 kernels (llama_generate_cpu_impl, "
                "temperature 0, no penalty, no EOS stop)",
        "model": {"arch": "LLaMA-2-7B", **LLAMA2_7B, "n_ctx": N_CTX, "weights": "SynthLlama seed 5, "
                  "N(0, 0.02) quantized Q4_K_M (Q6_K attn_v, ffn_down, output)"},
        "prompt_rule": "BOS = 1, then numpy default_rng(5).integers(0, n_vocab, 511)",
        "prompt": [int(t) for t in prompt],
        "ids": [int(t) for t in ids],
        "margins": [float(m) for m in margins],
        "top_ids": [[int(t) for t in r] for r in top_ids],
        "top_logits": [[float(v) for v in r] for r in top_vals],
        "isa": "AVX-VNNI" if O.ref.ref_has_avxvnni() else "AVX2",
        "seconds": round(dt, 1),
    }
    OUT.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {OUT} in {dt:.0f} s: ids {out['ids'][:8]} ..., min margin {min(out['margins']):.3e}",
          file=sys.stderr)
    return 0


if __name__ == "__main__":
    sys.exit(main())
