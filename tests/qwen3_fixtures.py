"""The transformers golden fixtures of tests/golden/ (written by
tests/golden/make_qwen3_golden.py) and the decode bar applied to them.

Bar: identical greedy tokens for the first 32 steps,
logits within 2e-2 max abs of transformers' Qwen3ForCausalLM (the
qwen3/reference.py:39-44 path).

Where the oracle (and so the GPU engine, which reproduces its logits rows
bit for bit) departs from transformers is pinned op by op in
tests/golden/qwen3_opdiff_<name>.json (tests/golden/qwen3_op_diff.py): fed
transformers' own bf16 inputs, the oracle's residual adds, SiLU.mul and RoPE
(formula and tables) return transformers' codes exactly, its RMSNorm does so
at every small shape and differs by one code in ~4e-6 of the 0.6B shape's
outputs (the FP32 sum of squares in another order); only the sums - GEMV rows
and the attention - differ in a small share of their outputs, and there each
side equals the FP64 result rounded to bf16 about equally often. So the
logit distance is the propagated FP32 summation order, not a rounding-point
mismatch. It exceeds 2e-2 on some steps of four fixtures, all of them with
large activations (norm gains 1 + N(0, 1) or the 28-layer 0.6B stack);
there transformers' own two paths (generate against one-position steps)
differ by a similar amount where they are comparable (0.040 and 0.123 at
the 0.6B shape).

Asserted per step of each fixture:
  * max |logit - transformers| over the full vocabulary <= 2e-2 for every
    step of the fixtures not in OPEN_GAP;
  * for the OPEN_GAP fixtures (an open parity gap): the number of steps
    within 2e-2 as recorded, and every step within the largest distance
    measured, so that any change that moves a step further away fails.
Tokens: a free-running fixture's first 32 greedy tokens equal both
transformers paths. A teacher-forced fixture (the oracle fed transformers'
step-path tokens, so that a near-tie cannot make the streams part) must
give transformers' token at every step where transformers' top-2 margin
exceeds twice that step's logit distance (no deviation of that size can
flip such a step); DECISIVE records how many steps that covers, and how
many steps give the same token in all.
"""
import hashlib
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = ["tiny", "tiny-varied", "small-varied", "small-varied-b", "small-untied", "qwen3-0.6b",
         "qwen3-0.6b-varied"]
VARIED = ["tiny-varied", "small-varied", "small-varied-b", "small-untied", "qwen3-0.6b-varied"]
FORCED = ["small-untied", "qwen3-0.6b-varied"]
BAR = 2e-2

# name: (steps of 32 within BAR, largest full-vocabulary distance measured)
OPEN_GAP = {
    "small-varied": (22, 0.03125),
    "small-untied": (31, 0.0234375),
    "qwen3-0.6b": (0, 0.04736328125),
    "qwen3-0.6b-varied": (0, 0.161865234375),
}

# teacher-forced fixtures: (decisive steps, steps with transformers' token)
DECISIVE = {"small-untied": (28, 31), "qwen3-0.6b-varied": (8, 28)}


def load(name):
    with open(os.path.join(GOLDEN, f"qwen3_{name}.json")) as fh:
        return json.load(fh)


def load_opdiff(name):
    with open(os.path.join(GOLDEN, f"qwen3_opdiff_{name}.json")) as fh:
        return json.load(fh)


def row_hash(codes) -> str:
    return hashlib.sha256(np.ascontiguousarray(codes, dtype="<u2").tobytes()).hexdigest()


def step_distance(st) -> float:
    """The step's max |oracle - transformers| against every transformers
    path whose row answers the same inputs (generate's rows after its stream
    parts from the step path's are recorded as None)."""
    return max(v for v in (st["oracle_vs_generate"], st["oracle_vs_steps"]) if v is not None)


def decisive(st) -> bool:
    return st["steps_margin"] > 2 * st["oracle_vs_steps"]


def forced_inputs(fx):
    """The token fed at each position of a teacher-forced fixture: the prompt,
    then transformers' step-path tokens."""
    return list(fx["prompt"]) + fx["hf_steps"][:fx["logit_steps"] - 1]
