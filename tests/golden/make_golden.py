"""Writes tests/golden/ref_vectors.npz and ref_vectors.json from the compiled reference.

Run in the container that holds /root/reference, after ``make -C oracle``:

    python tests/golden/make_golden.py

Every expected value comes from oracle/_ref/libkvexp_ref.so, i.e. the reference
library (src/codec.cpp, src/dispatch.cpp, src/attention_*.cpp) compiled from its
own sources. Inputs are seeded and regenerated here. The fixtures are data only:
inputs, containers and outputs, with a SHA-256 of every container.

Cases:
  codec/*   containers from encode_bf16 (codec.cpp:39-164), including the
            reference unit-test inputs (tests/test_main.cpp:54-86) and the
            size-tie corner cases of codec.cpp:94-103.
  attn/*    attention_decode outputs (dispatch.cpp:27-104) for the scalar, AVX2
            and AVX-512 BF16 backends; raw and XKV outputs are asserted equal
            before they are stored.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

from oracle import Reference  # noqa: E402
from kvdata import bf16_from_f32, random_kv, ref_test_stream  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def tie_cases():
    """Blocks whose candidate container sizes tie (codec.cpp:94-103)."""
    one = 0x3F80  # exponent 127
    out = []
    # n=2, dim=4, each channel's two exponents 5 apart: 2-bit has 4 escapes (30 B),
    # 4-bit has none (24 B) and ties raw (24 B) -> raw.
    kv = np.array([127 << 7] * 4 + [132 << 7] * 4, np.uint16)
    out.append(("tie_raw_vs_4bit", 2, 4, 2, kv))
    # n=2, dim=4, one value outside the 2-bit window: 2-bit = 24 B = raw -> raw.
    kv = np.full(8, one, np.uint16)
    kv[3] = 0x4780  # exponent 143
    out.append(("tie_raw_vs_2bit", 2, 4, 2, kv))
    # n=8, dim=4: 2-bit misses 4 values (60 B), 4-bit misses none (60 B), raw 72 B -> 4-bit.
    kv = np.full(32, one, np.uint16)
    for i, e in enumerate((130, 131, 132, 133)):
        kv[4 * i] = (e << 7)
    out.append(("tie_2bit_vs_4bit", 8, 4, 8, kv))
    # Smallest-base tie: channel 0 holds exponents 100,100,200,200 -> two windows
    # of count 2; the smallest maximising base (98 for 2-bit) wins.
    kv = np.full(16, 0x3F80, np.uint16)
    for t, e in enumerate((100, 100, 200, 200)):
        kv[4 * t] = e << 7
    out.append(("tie_base_choice", 4, 4, 4, kv))
    return out


def main() -> None:
    R = Reference()
    if not R.avx512_bf16:
        raise SystemExit("an AVX512_BF16 host is needed to write the AVX-512 fixtures")
    arrays: dict[str, np.ndarray] = {}
    manifest: dict[str, list] = {"codec": [], "attn": []}

    def add_codec(name, kv, seq, dim, block):
        blob = R.encode(kv, seq, dim, block)
        dec = R.decode(blob, seq, dim)
        assert np.array_equal(dec, kv.reshape(-1)), name
        arrays[f"codec/{name}/kv"] = kv.reshape(-1)
        arrays[f"codec/{name}/blob"] = blob
        manifest["codec"].append(dict(name=name, seq=seq, dim=dim, block=block, bytes=int(blob.size),
                                      sha256=sha(blob)))

    def add_attn(name, q, k, v, n_q, dim, seq, block, threads_list, backends=("scalar", "avx2", "avx512")):
        kx = R.encode(k, seq, dim, block)
        vx = R.encode(v, seq, dim, block)
        arrays[f"attn/{name}/q"] = q
        arrays[f"attn/{name}/k"] = k
        arrays[f"attn/{name}/v"] = v
        entry = dict(name=name, n_q=n_q, dim=dim, seq=seq, block=block, threads=list(threads_list),
                     k_sha256=sha(kx), v_sha256=sha(vx), backends=[])
        for be in backends:
            if be == "avx512" and dim % 32:
                continue
            entry["backends"].append(be)
            for th in threads_list:
                raw = R.attention(be, q, k, v, n_q=n_q, dim=dim, seq=seq, threads=th, split=block)
                xkv = R.attention(be, q, kx=kx, vx=vx, n_q=n_q, dim=dim, seq=seq, threads=th, split=block)
                assert np.array_equal(raw.view(np.uint32), xkv.view(np.uint32)), (name, be, th)
                arrays[f"attn/{name}/{be}/t{th}"] = raw
        manifest["attn"].append(entry)

    # -- the reference unit-test inputs --------------------------------------
    for item in ref_test_stream():
        if item[0] == "roundtrip":
            _, block, kv = item
            add_codec(f"ref_roundtrip_b{block}", kv, 300, 64, block)
        elif item[0] == "size":
            add_codec("ref_size_formula", item[1], 128, 64, 128)
        else:
            _, (dim, n_q, seq, block, th), q, k, v = item
            add_attn(f"ref_bitexact_d{dim}_q{n_q}_s{seq}_b{block}_t{th}", q, k, v, n_q, dim, seq, block,
                     sorted({1, th}))

    # -- size-tie and base-tie corner cases ----------------------------------
    for name, seq, dim, block, kv in tie_cases():
        add_codec(name, kv, seq, dim, block)

    rng = np.random.default_rng(20261201)
    # -- mode coverage: 2-bit and raw blocks, wide dims, block 255 --------------
    x = rng.uniform(1.0, 7.9, 256 * 64).astype(np.float32) * np.where(rng.random(256 * 64) < .5, -1, 1)
    add_codec("bits2_dim64", bf16_from_f32(x), 256, 64, 128)
    kv = rng.integers(0, 65536, 200 * 32, dtype=np.uint16)
    add_codec("raw_dim32", kv, 200, 32, 64)
    add_codec("dim256_block255", random_kv(rng, 300, 256, specials=True, wide=True), 300, 256, 255)
    add_codec("dim128_mixed", random_kv(rng, 333, 128, outliers=3, specials=True), 333, 128, 128)
    add_codec("dim4_block1", random_kv(rng, 7, 4), 7, 4, 1)
    add_codec("dim12_ragged", random_kv(rng, 50, 12, wide=True), 50, 12, 16)

    # -- attention coverage ------------------------------------------------------
    def qk(n, d):
        return random_kv(rng, n, d, spread_lo=-1, spread_hi=1)

    # Config-1-like micro case (dim 64, 1 query), shortened to keep the fixture small.
    add_attn("c1_like_d64_q1_s2048", qk(1, 64), random_kv(rng, 2048, 64), random_kv(rng, 2048, 64, sigma=0.5),
             1, 64, 2048, 128, [1, 4, 16])
    # Qwen-like GQA group of 7 with outlier channels and 2-bit blocks.
    kx = random_kv(rng, 1000, 64, spread_lo=-6, spread_hi=4, outliers=2)
    band = bf16_from_f32((rng.uniform(1.0, 7.9, 128 * 64) * np.where(rng.random(128 * 64) < .5, -1, 1)).astype(np.float32))
    kx[128 * 64:256 * 64] = band
    add_attn("qwen_like_d64_q7_s1000", qk(7, 64), kx, random_kv(rng, 1000, 64, sigma=0.5), 7, 64, 1000, 128,
             [1, 3, 8])
    # Llama-like dim 128, group 4.
    add_attn("llama_like_d128_q4_s700", qk(4, 128), random_kv(rng, 700, 128, spread_lo=-5, spread_hi=3),
             random_kv(rng, 700, 128, sigma=0.5), 4, 128, 700, 128, [1, 2, 6])
    # Edge: dim 256, block 255, group 8, specials in K and V, wide spread (raw / 2-bit / 4-bit mix).
    add_attn("edge_d256_q8_s600_b255", qk(8, 256), random_kv(rng, 600, 256, specials=True, wide=True),
             random_kv(rng, 600, 256, specials=True), 8, 256, 600, 255, [1, 3])
    # Raw-mode blocks inside attention.
    kraw = rng.integers(0, 65536, 300 * 32, dtype=np.uint16)
    kraw[(kraw & 0x7F80) == 0x7F80] &= 0x3FFF
    add_attn("rawmode_d32_q2_s300_b64", qk(2, 32), kraw, random_kv(rng, 300, 32), 2, 32, 300, 64, [1, 5])
    # dim 8 / 24 (scalar and AVX2 only), single token, odd groups.
    add_attn("d8_q3_s1", qk(3, 8), random_kv(rng, 1, 8), random_kv(rng, 1, 8), 3, 8, 1, 128, [1],
             backends=("scalar", "avx2"))
    add_attn("d24_q5_s77_b16", qk(5, 24), random_kv(rng, 77, 24), random_kv(rng, 77, 24), 5, 24, 77, 16, [1, 4],
             backends=("scalar", "avx2"))

    npz = os.path.join(HERE, "ref_vectors.npz")
    np.savez_compressed(npz, **arrays)
    with open(os.path.join(HERE, "ref_vectors.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    print(f"wrote {npz} ({os.path.getsize(npz)} bytes), {len(manifest['codec'])} codec and "
          f"{len(manifest['attn'])} attention cases")


if __name__ == "__main__":
    main()
