"""The oracle's encoder and the KVD1 reader against fixtures written by the
reference's own numpy code (python/analyze_exponents.py, via
tests/golden/make_analyze_golden.py): for every exponent field, the
container that encode_bf16's policy (2- and 4-bit) and the 3-bit extension
(2-, 3- and 4-bit) produce has the size, the block modes and the escape count
that the reference's policy_size (analyze_exponents.py:117-157) computes;
dumps.parse_dump reads a KVD1 file into the planes and header that the
reference's load_dump (analyze_exponents.py:23-32) reads."""
import json
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def analyze():
    z = np.load(os.path.join(HERE, "golden", "analyze_vectors.npz"), allow_pickle=False)
    with open(os.path.join(HERE, "golden", "analyze_vectors.json")) as f:
        return z, json.load(f)


def _escapes(oracle, blob, dim, seq):
    """Escape count summed over the container's block headers."""
    off, _ = oracle.block_index(blob, dim, seq)
    return int(sum(int(blob[o + 2]) | (int(blob[o + 3]) << 8) for o in off[:-1]))


def test_encoder_matches_reference_sizer(oracle, analyze):
    z, man = analyze
    assert len(man["size"]) >= 12
    for c in man["size"]:
        bits = z[f"size/{c['name']}/bits"].reshape(-1)
        modes = 0x1C if 3 in c["widths"] else 0x14
        blob = oracle.encode(bits, c["seq"], c["dim"], c["block"], modes=modes)
        what = (c["name"], tuple(c["widths"]))
        assert blob.size == c["container_bytes"], what
        counts = oracle.mode_counts(blob, c["dim"])
        got = {str(m): counts[m] for m in range(5) if counts[m]}
        assert got == c["mode_blocks"], what
        assert _escapes(oracle, blob, c["dim"], c["seq"]) == c["escapes"], what
        assert 2 * c["seq"] * c["dim"] == c["tight_bytes"]


def test_dump_reader_matches_reference_reader(analyze, tmp_path):
    import sys

    sys.path.insert(0, os.path.join(os.path.dirname(HERE), "compressed-kv-attention_amd"))
    from kvexp_amd import dumps

    z, man = analyze
    assert man["dump"]
    for c in man["dump"]:
        path = tmp_path / f"{c['name']}.kvd"
        z[f"dump/{c['name']}/file"].tofile(path)
        d = dumps.parse_dump(str(path))
        assert (d.layers, d.kv, d.nq, d.dim, d.seq) == (
            c["n_layers"], c["n_kv_heads"], c["n_q_heads"], c["head_dim"], c["seq_len"])
        assert np.array_equal(np.asarray(d.k), z[f"dump/{c['name']}/k"])
        assert np.array_equal(np.asarray(d.v), z[f"dump/{c['name']}/v"])
