"""Writes tests/golden/seed_golden.json: input/output vectors of the reference's
own `_next_seed()` (reference @ None: flash_attn_v100_cuda.py:28-33).

The seed counter is the one function of the hot path that no library routine,
closed-form property or published algorithm pins: it is a formula of the
reference's own.  So this script imports the reference module itself, in the
build container only, and records what it returns:

  * the module is loaded by file path under another name
    (`ref_flash_attn_v100_cuda`), so it cannot be mistaken for the drop-in
    module; importing it runs no build (the reference compiles its extension
    lazily, in `_build()`, which `_next_seed` does not call);
  * `torch.cuda.initial_seed` is replaced by a function returning each test
    value in turn (the reference looks it up at call time), including values
    of 2^32 and above (`initial_seed` is a 64-bit seed);
  * the module's `_SEED_COUNTER` is reset to `itertools.count(1)` before each
    value, as in a fresh process, and `_next_seed()` is called five times.

Only the numbers are written; nothing of the reference is kept.  Run:
    python tests/golden/make_seed_golden.py
"""
import importlib.util
import itertools
import json
import os

import torch

REF = os.environ.get("FA2_REFERENCE", "/root/reference")
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "seed_golden.json")

# initial_seed values: small, around 2^31 and 2^32, 64-bit, and torch's
# default-style large seeds.
INITIAL_SEEDS = [0, 1, 2, 42, 12345, 2 ** 31 - 1, 2 ** 31, 2 ** 32 - 1, 2 ** 32, 2 ** 32 + 1,
                 2 ** 40 + 3, 67280421310721, 2 ** 63 - 1, 2 ** 64 - 1]
CALLS = 5


def main():
    path = os.path.join(REF, "flash_attn_v100_cuda.py")
    spec = importlib.util.spec_from_file_location("ref_flash_attn_v100_cuda", path)
    ref = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(ref)
    saved = torch.cuda.initial_seed
    cases = []
    try:
        for s in INITIAL_SEEDS:
            torch.cuda.initial_seed = (lambda v=s: v)
            ref._SEED_COUNTER = itertools.count(1)
            cases.append({"initial_seed": s, "seeds": [int(ref._next_seed()) for _ in range(CALLS)]})
    finally:
        torch.cuda.initial_seed = saved
    with open(OUT, "w") as f:
        json.dump({"source": "flash_attn_v100_cuda.py:28-33 (_next_seed), imported from the reference",
                   "cases": cases}, f, indent=1)
    print(f"wrote {OUT}: {len(cases)} initial seeds x {CALLS} calls")


if __name__ == "__main__":
    main()
