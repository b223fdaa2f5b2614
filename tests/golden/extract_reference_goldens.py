"""Writes reference_goldens.json: the golden values of the reference's own test-suite that pin this build's oracle.

It reads tests/golden_values.py of the reference checkout as text (ast.literal_eval on its constant assignments; the
module is never imported or executed) and keeps the tables the fine-tuning path can reproduce. Run it where the
reference checkout exists; the committed JSON is what tests read.
"""

from __future__ import annotations

import ast
import json
import sys
from pathlib import Path

KEEP = ("RANDOM_FIRST", "RANDOM_SECOND", "KERNEL_FINGERPRINTS", "GRADIENT_FINGERPRINT", "FINETUNE_FINGERPRINT",
        "LORA_FINETUNE_FINGERPRINT", "DPO_FINETUNE_FINGERPRINT", "LONG_CONTEXT_FINGERPRINTS",
        "TINY_LOGITS_FINGERPRINT", "QLORA_FINETUNE_FINGERPRINT")


def main(reference: Path, out: Path) -> None:
    tree = ast.parse((reference / "tests" / "golden_values.py").read_text(encoding="utf-8"))
    values = {}
    for node in tree.body:
        if isinstance(node, ast.Assign) and len(node.targets) == 1 and isinstance(node.targets[0], ast.Name):
            name = node.targets[0].id
            if name in KEEP:
                values[name] = ast.literal_eval(node.value)
    values["_source"] = "reference tests/golden_values.py (RUN configs: tests/test_training.py:32,50,357)"
    out.write_text(json.dumps(values, indent=1, sort_keys=True) + "\n", encoding="utf-8")


if __name__ == "__main__":
    ref = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference")
    main(ref, Path(__file__).with_name("reference_goldens.json"))
