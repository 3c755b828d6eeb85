#!/usr/bin/env python3
"""Converts llm-shield's real-model activation fixture into a compact array file.

Reads tests/fixtures/activations.json of the reference (captured from its NumPy
implementation on the original Shieldstral weights, see its ActivationParityTests.cs):
the prompt's 80 token ids, and for each recorded tensor its shape, last row and
squared Frobenius norm; the top-20 logits of the last position. Writes the same data
unchanged (float32 rows, float64 norms) into tests/golden/real_model_activations.npz.
Run in the container that has the reference mounted:

    python3 tests/golden/extract_activation_fixture.py /root/reference/tests/fixtures/activations.json
"""
import json
import sys
from pathlib import Path

import numpy as np


def main() -> int:
    src = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/tests/fixtures/activations.json")
    data = json.loads(src.read_text())
    names = list(data["tensors"])
    arrays = {
        "tokens": np.asarray(data["tokens"], np.int32),
        "names": np.asarray(names),
        "rows": np.asarray([data["tensors"][n]["rows"] for n in names], np.int32),
        "columns": np.asarray([data["tensors"][n]["columns"] for n in names], np.int32),
        "checksum": np.asarray([data["tensors"][n]["checksum"] for n in names], np.float64),
        "top20": np.asarray(data["logits"]["top20"], np.int32),
        # logits of the top-20 ids, keyed by id in the JSON
        "top20_values": np.asarray([data["logits"]["values"][str(t)] for t in data["logits"]["top20"]], np.float32),
    }
    for i, n in enumerate(names):
        row = np.asarray(data["tensors"][n]["last_row"], np.float64)
        assert np.array_equal(row.astype(np.float32).astype(np.float64), row), n  # float32 values, kept exactly
        arrays[f"last_row_{i}"] = row.astype(np.float32)
    out = Path(__file__).resolve().parent / "real_model_activations.npz"
    np.savez_compressed(out, **arrays)
    print(f"wrote {out} ({len(names)} tensors, {out.stat().st_size} bytes)")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
