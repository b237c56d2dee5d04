"""Extracts golden values from the reference's two training logs.

Reads (as text) output-DiZO-SST2.log and output-MeZO-SST2.log from the
reference checkout and writes tests/golden/reference_log.json with:
  * every logged (global_step, lr) pair -- the ZO LambdaLR schedule of
    trainer.py:1100-1102 with LR 1e-6 and max_steps 4000 (logged every 50
    steps by trainer.py:1321-1325);
  * the logged "Number of trainable parameters" of OPT-2.7B;
  * the logged losses of both runs (DiZO == MeZO until the first projection).

Run: python tests/golden/make_reference_log_fixtures.py [/root/reference]
"""
from __future__ import annotations

import ast
import json
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def parse(path):
    text = open(path, encoding="utf-8", errors="replace").read()
    entries = [ast.literal_eval(m) for m in re.findall(r"\{'loss'[^}]*\}", text)]
    m = re.search(r"Number of trainable parameters = (\d+)", text)
    steps = re.search(r"Total optimization steps = (\d+)", text)
    return entries, int(m.group(1)), int(steps.group(1))


def main(ref_root="/root/reference"):
    out = {}
    for tag, name in (("dizo", "output-DiZO-SST2.log"), ("mezo", "output-MeZO-SST2.log")):
        entries, nparams, max_steps = parse(os.path.join(ref_root, name))
        out[tag] = {
            "max_steps": max_steps,
            "trainable_parameters": nparams,
            # logging happens every 50 global steps (trainer.py:1320-1325)
            "log": [{"global_step": 50 * (i + 1), "loss": e["loss"], "lr": e["lr"]}
                    for i, e in enumerate(entries)],
        }
    out["learning_rate"] = 1e-6
    out["source"] = "tests/golden/make_reference_log_fixtures.py"
    with open(os.path.join(HERE, "reference_log.json"), "w") as f:
        json.dump(out, f, indent=1)
    print({k: len(v["log"]) for k, v in out.items() if isinstance(v, dict)})


if __name__ == "__main__":
    main(*sys.argv[1:])
