"""Writes tests/golden/analyze_vectors.npz and analyze_vectors.json from the
reference's own numpy code, python/analyze_exponents.py, imported from
/root/reference in the container that holds it:

    python tests/golden/make_analyze_golden.py

The reference's C++ never writes 3-bit blocks; its only statement of the
3-bit choice is the sizer in analyze_exponents.py (policy_size, :117-157),
and its KVD1 reader there (load_dump, :23-32) is the other half of the dump
format beside bench.cpp's parse_dump. This script runs both on seeded inputs
and stores inputs and outputs only (no code):

  size/<case>/<widths>  BF16 bits [seq, dim] -> policy_size(exp, block, widths):
                        container bytes, tight bytes, escape count, block modes
  dump/<case>           a small KVD1 file's bytes -> load_dump's K, V planes and
                        header fields
"""
from __future__ import annotations

import json
import os
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF_PY = "/root/reference/python"
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, os.path.join(ROOT, "compressed-kv-attention_amd"))
sys.path.insert(0, REF_PY)

import analyze_exponents as ax  # noqa: E402  (the reference's module, read-only)
from kvdata import random_kv  # noqa: E402
from kvexp_amd import dumps, synth  # noqa: E402


def size_cases():
    rng = np.random.default_rng(2024)
    k, v = synth.head_kv("c2", 4096, 0, 3, 1)
    k5, _ = synth.head_kv("c5", 765, 0, 0, 2)
    return [
        ("c2_k", k.reshape(4096, 64), 128),
        ("c2_v", v.reshape(4096, 64), 128),
        ("wide", random_kv(rng, 1000, 64, wide=True).reshape(1000, 64), 128),
        ("dim128", random_kv(rng, 700, 128, spread_lo=-5, spread_hi=3).reshape(700, 128), 100),
        ("c5_dim256", k5.reshape(765, 256), 255),
        ("tail", random_kv(rng, 130, 64, specials=True).reshape(130, 64), 128),
    ]


def main() -> None:
    arrays, manifest = {}, {"size": [], "dump": []}
    for name, bits, block in size_cases():
        exp = ((bits >> 7) & 0xFF).astype(np.uint8)
        arrays[f"size/{name}/bits"] = bits.astype(np.uint16)
        for widths in ((2, 4), (2, 3, 4)):
            r = ax.policy_size(exp, block, widths)
            seq, dim = bits.shape
            manifest["size"].append({
                "name": name, "seq": seq, "dim": dim, "block": block, "widths": list(widths),
                "container_bytes": r["container_bytes"], "tight_bytes": r["tight_bytes"],
                "escapes": int(round(r["escape_rate"] * seq * dim)),
                "mode_blocks": r["mode_blocks"],
            })
    rng = np.random.default_rng(77)
    for name, (layers, kv, nq, dim, seq) in {"small": (2, 2, 4, 8, 16), "odd": (1, 3, 6, 12, 5)}.items():
        k = rng.integers(0, 1 << 16, (layers, kv, seq, dim), dtype=np.uint16)
        v = rng.integers(0, 1 << 16, (layers, kv, seq, dim), dtype=np.uint16)
        q = rng.integers(0, 1 << 16, (layers, nq, dim), dtype=np.uint16)
        with tempfile.TemporaryDirectory() as d:
            path = os.path.join(d, "x.kvd")
            dumps.write_dump(path, k, v, q)
            raw = np.fromfile(path, dtype=np.uint8)
            rk, rv, meta = ax.load_dump(Path(path))
        arrays[f"dump/{name}/file"] = raw
        arrays[f"dump/{name}/k"] = rk
        arrays[f"dump/{name}/v"] = rv
        manifest["dump"].append({"name": name, **{key: int(val) for key, val in meta.items()}})
    np.savez_compressed(os.path.join(HERE, "analyze_vectors.npz"), **arrays)
    with open(os.path.join(HERE, "analyze_vectors.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    print(f"wrote {len(manifest['size'])} size cases and {len(manifest['dump'])} dumps")


if __name__ == "__main__":
    main()
