"""The composition tests catch wiring slips in the oracle's decoder.

Each case below plants one slip in a copy of oracle/axf_oracle.c (an exact
text edit of one statement), builds it with the Makefile's flags, and runs
tests/test_oracle_compose.py and tests/test_oracle_compose_types.py against
that build (oracle.py loads it through AXF_ORACLE_LIB).  Every mutant must
fail at least one test; the unmutated copy, built the same way, must pass.
The slips are the ones a restatement of llama_forward_token /
llama_forward_batch / llama_generate_cpu_impl (src/models/llama_model.cpp:
1207-1333, 1339-1462, 1561-1624) can plausibly get wrong; each is written so
the mutant stays memory-safe (a slip that would index past a buffer is
replaced by its in-bounds neighbour).  CPU only.
"""
import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
SRC = ROOT / "oracle" / "axf_oracle.c"
TESTS = ["tests/test_oracle_compose.py", "tests/test_oracle_compose_types.py"]
CFLAGS = ["-O3", "-mavx2", "-mfma", "-ffp-contract=off", "-fPIC", "-std=c11", "-shared"]

# (name, statement in axf_oracle.c, replacement)
MUTANTS = [
    ("K row stored without RoPE (decode)",
     "orc_rope(krow, s->k, pos, KVH, HD, s->rope_cos, s->rope_sin);",
     "memcpy(krow, s->k, sizeof(float) * (size_t)KVH * HD);"),
    ("FFN norm with attn_norm (decode)",
     "orc_rmsnorm(s->xb, s->x, lw->ffn_norm, E, m->rms_eps);",
     "orc_rmsnorm(s->xb, s->x, lw->attn_norm, E, m->rms_eps);"),
    ("k bias dropped (decode)",
     "add_bias(s->k, lw->bk, KVH * HD);",
     "(void)0;"),
    ("FFN residual dropped (decode)",
     "for (int i = 0; i < E; i++) s->x[i] += s->ffn[i];",
     "(void)0;"),
    ("final norm dropped (decode)",
     "orc_rmsnorm(s->x, s->x, m->output_norm, E, m->rms_eps);",
     "(void)0;"),
    ("final norm dropped (batch)",
     "orc_rmsnorm(xl, xl, m->output_norm, E, m->rms_eps);",
     "(void)0;"),
    ("gate and up swapped in SwiGLU (decode)",
     "orc_swiglu(s->gate, s->up, FD);",
     "orc_swiglu(s->up, s->gate, FD); memcpy(s->gate, s->up, sizeof(float) * (size_t)FD);"),
    ("attention over pos rows instead of pos + 1 (decode)",
     "orc_attention(s->attn_out, s->q, kc, vc, pos + 1, H, KVH, HD, s->attn);",
     "orc_attention(s->attn_out, s->q, kc, vc, pos > 0 ? pos : 1, H, KVH, HD, s->attn);"),
    ("kv head of query head h is h % KVH",
     "const int kvh = h / group;",
     "const int kvh = h % n_kv_heads;"),
    ("generation stops one step before the context end",
     "if (n_past >= m->n_ctx) break;",
     "if (n_past + 1 >= m->n_ctx) break;"),
    ("query rotated at pos + 1 (decode)",
     "orc_rope(s->q, s->q, pos, H, HD, s->rope_cos, s->rope_sin);",
     "orc_rope(s->q, s->q, (pos + 1) % m->n_ctx, H, HD, s->rope_cos, s->rope_sin);"),
    ("batched K rotated at the row index, not the position",
     "orc_rope(krow, K + (size_t)t * kve, pos, KVH, HD, s->rope_cos, s->rope_sin);",
     "orc_rope(krow, K + (size_t)t * kve, t, KVH, HD, s->rope_cos, s->rope_sin);"),
    ("first generated token taken from the prompt",
     "int next = orc_argmax(s->logits, m->n_vocab);",
     "int next = prompt[n_prompt - 1];"),
]


def _build_and_run(tmp: Path, tag: str, edit):
    src = SRC.read_text()
    if edit is not None:
        old, new = edit
        assert src.count(old) == 1, f"{tag}: the statement to mutate is not unique in axf_oracle.c"
        src = src.replace(old, new)
    d = tmp / tag
    d.mkdir()
    (d / "axf_oracle.c").write_text(src)
    (d / "axf_oracle.h").write_text((SRC.parent / "axf_oracle.h").read_text())
    lib = d / "liboracle.so"
    cc = subprocess.run(["gcc", *CFLAGS, "-o", str(lib), str(d / "axf_oracle.c"), "-lm"],
                        capture_output=True, text=True)
    assert cc.returncode == 0, f"{tag}: build failed\n{cc.stderr}"
    env = dict(os.environ, AXF_ORACLE_LIB=str(lib))
    run = subprocess.run([sys.executable, "-m", "pytest", *TESTS, "-x", "-q", "-p", "no:cacheprovider",
                          "-m", "not gpu"], cwd=ROOT, env=env, capture_output=True, text=True,
                         timeout=600)
    return run.returncode, run.stdout[-2000:]


@pytest.mark.slow
def test_every_planted_slip_fails_a_composition_test():
    with tempfile.TemporaryDirectory() as t:
        tmp = Path(t)
        rc, out = _build_and_run(tmp, "unmutated", None)
        assert rc == 0, f"the unmutated copy must pass:\n{out}"
        with ThreadPoolExecutor(max_workers=4) as ex:
            res = list(ex.map(lambda im: _build_and_run(tmp, f"m{im[0]}", im[1][1:]), enumerate(MUTANTS)))
        survived = [MUTANTS[i][0] for i, (rc, _) in enumerate(res) if rc == 0]
        for (name, _, _), (rc, _) in zip(MUTANTS, res):
            print(f"  {'caught  ' if rc else 'SURVIVED'}  {name}")
        assert not survived, f"slips no test caught: {survived}"
