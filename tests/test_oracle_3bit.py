"""The 3-bit format extension in the oracle (CPU).

The reference sizes a 3-bit mode (python/analyze_exponents.py:104-157) but
its encoder, readers and kernels do not implement it, so there is no
reference output to compare with. What pins the oracle here:
* a hand-packed block read back through the oracle's decoder, with the code
  stream built as one Python integer (element i at bits [3i, 3i + 3));
* decode(encode(x)) == x with the extension allowed, and the reference's
  containers unchanged without it;
* a restatement of the reference's sizer (per block: candidates raw / 2 / 3 /
  4 bits, sizes by the byte formula, min by size, raw, escapes, bits) that
  must give each block's mode, escape count and byte size, and numpy's first
  argmax of the window counts that must give each base (best_base's
  smallest maximiser, codec.cpp:18-35).
"""
import numpy as np
import pytest

from kvdata import random_kv

MODES_REF = 0x14
MODES_3BIT = 0x1C


def _blocks(blob, dim):
    """(mode, n_tokens, n_escape, offset, size) per block from the headers."""
    out, p = [], 0
    while p < blob.size:
        mode, n = int(blob[p]), int(blob[p + 1])
        esc = int(blob[p + 2]) | (int(blob[p + 3]) << 8)
        size = 8 + 2 * n * dim if mode == 0 else 8 + dim + n * dim + (n * dim * mode + 7) // 8 + 2 * esc
        out.append((mode, n, esc, p, size))
        p += size
    assert p == blob.size
    return out


def _sizer(exp, block, bit_widths):
    """analyze_exponents.py:117-143 per block: (mode, bytes, n_escape) and the
    window bases per width."""
    seq, dim = exp.shape
    res = []
    for start in range(0, seq, block):
        piece = exp[start:start + block].astype(np.int64)
        n = piece.shape[0]
        hist = np.zeros((dim, 256), np.int64)
        np.add.at(hist, (np.broadcast_to(np.arange(dim), piece.shape), piece), 1)
        csum = np.cumsum(hist, axis=1)
        pad = np.concatenate([np.zeros((dim, 1), np.int64), csum], axis=1)
        options, bases = [(0, 8 + 2 * n * dim, 0)], {}
        for bits in bit_widths:
            width = (1 << bits) - 1
            b = np.arange(256 - width + 1)
            cnt = csum[:, b + width - 1] - pad[:, b]
            n_esc = int(n * dim - cnt.max(axis=1).sum())
            options.append((bits, 8 + dim + n * dim + (n * dim * bits + 7) // 8 + 2 * n_esc, n_esc))
            bases[bits] = cnt.argmax(axis=1)  # first maximiser = smallest base
        res.append((min(options, key=lambda t: (t[1], 0 if t[0] == 0 else 1, t[2], t[0])), bases))
    return res


def test_3bit_reader_kat(oracle):
    """A mode-3 block built by hand: dim 8, 2 tokens, codes 0..7 then 6..0, 7
    (two sentinels, so two escape words in scan order)."""
    dim, n = 8, 2
    base = np.arange(100, 108, dtype=np.uint8)
    rng = np.random.default_rng(31)
    sm = rng.integers(0, 256, n * dim, dtype=np.uint8)
    codes = [0, 1, 2, 3, 4, 5, 6, 7, 6, 5, 4, 3, 2, 1, 0, 7]
    stream = sum(c << (3 * i) for i, c in enumerate(codes)).to_bytes(6, "little")
    esc = np.array([0x1234, 0xBEEF], dtype="<u2")
    hdr = bytes([3, n, 2, 0, dim, 0, 0, 0])
    blob = np.frombuffer(hdr + base.tobytes() + sm.tobytes() + stream + esc.tobytes(), dtype=np.uint8)
    want, e = [], 0
    for i, c in enumerate(codes):
        if c == 7:
            want.append(int(esc[e]))
            e += 1
        else:
            s = int(sm[i])
            want.append(((s & 0x80) << 8) | (((int(base[i % dim]) + c) & 0xFF) << 7) | (s & 0x7F))
    assert oracle.decode(blob, n, dim).tolist() == want
    assert oracle.mode_counts(blob, dim) == [0, 0, 0, 1, 0]
    # the reference's readers reject mode 3; so does the oracle when the rows
    # would not start on a byte (head_dim not a multiple of 8)
    bad = np.frombuffer(bytes([3, 1, 0, 0, 12, 0, 0, 0]) + bytes(12 + 12 + 5), dtype=np.uint8)
    with pytest.raises(Exception, match="unknown xkv block mode"):
        oracle.decode(bad, 1, 12)


@pytest.mark.parametrize("trial", range(24))
def test_3bit_roundtrip_and_sizer(oracle, trial):
    rng = np.random.default_rng(300 + trial)
    dim = 8 * int(rng.integers(1, 33)) if trial % 4 else 4 * int(rng.integers(1, 65))
    seq = int(rng.integers(1, 600))
    block = int(rng.integers(1, min(255, 65535 // dim) + 1))
    if trial % 3 == 0:
        kv = random_kv(rng, seq, dim, specials=True, wide=trial % 6 == 0)
    elif trial % 3 == 1:  # exponents in narrow windows: 2-, 3- and 4-bit all compete, many ties
        exp = rng.integers(0, 256, dim)[None, :] + rng.integers(0, int(rng.integers(2, 12)), (seq, dim))
        kv = ((np.clip(exp, 0, 255) << 7) | rng.integers(0, 128, (seq, dim))
              | (rng.integers(0, 2, (seq, dim)) << 15)).astype(np.uint16).reshape(-1)
    else:
        kv = random_kv(rng, seq, dim, spread_lo=-1.0, spread_hi=1.0)
    ref = oracle.encode(kv, seq, dim, block)
    assert np.array_equal(oracle.encode(kv, seq, dim, block, modes=MODES_REF), ref)
    blob = oracle.encode(kv, seq, dim, block, modes=MODES_3BIT)
    assert np.array_equal(oracle.decode(blob, seq, dim), kv)
    assert blob.size <= ref.size
    off, first = oracle.block_index(blob, dim, seq)
    assert first[-1] == seq and off[-1] == blob.size
    exp = ((kv.reshape(seq, dim) >> 7) & 0xFF).astype(np.uint8)
    widths = (2, 3, 4) if dim % 8 == 0 else (2, 4)
    blocks = _blocks(blob, dim)
    sized = _sizer(exp, block, widths)
    assert len(blocks) == len(sized)
    for (mode, n, esc, p, size), ((smode, sbytes, sesc), bases) in zip(blocks, sized):
        assert (mode, size) == (smode, sbytes)
        if mode:
            assert esc == sesc
            assert np.array_equal(blob[p + 8:p + 8 + dim], bases[mode].astype(np.uint8))
    if dim % 8:
        assert np.array_equal(blob, ref)  # the extension needs byte-aligned rows


def test_3bit_wins_on_narrow_exponents(oracle):
    """Exponents in a 7-wide window per channel: every block is 3-bit with no
    escape (8 + 64 + 8192 + 3072 = 11336 bytes at 128 x 64)."""
    rng = np.random.default_rng(33)
    exp = rng.integers(100, 107, 128 * 64)
    kv = ((exp << 7) | rng.integers(0, 128, exp.size)).astype(np.uint16)
    blob = oracle.encode(kv, 128, 64, 128, modes=MODES_3BIT)
    assert blob.size == oracle.coded_block_bytes(128, 64, 3, 0) == 11336
    assert oracle.mode_counts(blob, 64) == [0, 0, 0, 1, 0]
    assert np.array_equal(oracle.decode(blob, 128, 64), kv)


def test_reference_rejects_3bit(oracle, reference):
    """The deliberate difference: the reference's parse_block (scan.hpp:28-66)
    rejects mode 3, which the oracle (and the library) read."""
    from oracle import KvexpError

    rng = np.random.default_rng(34)
    exp = rng.integers(100, 107, 64 * 64)
    kv = ((exp << 7) | rng.integers(0, 128, exp.size)).astype(np.uint16)
    blob = oracle.encode(kv, 64, 64, 128, modes=MODES_3BIT)
    assert np.array_equal(oracle.decode(blob, 64, 64), kv)
    with pytest.raises(KvexpError, match="unknown xkv block mode"):
        reference.decode(blob, 64, 64)
