"""Writes tests/golden/ref_vectors.npz from the reference's own code.

    python oracle/build_ref.sh && python tests/golden/make_golden.py

Every expected value here comes out of run.cpp itself, compiled from the
reference sources by oracle/build_ref.sh (oracle/_ref/libref.so, this
container only): compute_cos_sin (run.cpp:479-504), apply_rotary_emb
(run.cpp:506-526), softmax (run.cpp:335-353) and forward()'s attention on a
synthetic single-sequence model (run.cpp:528-642, see oracle/ref_harness.cpp).

Inputs are seeded random numbers. History keys/values are bf16-representable
floats (stored as their 16-bit patterns), which is also what the bf16 cache
holds; the new token's q|k|v row is full fp32.
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import kv_oracle as O  # noqa: E402

SEED = 20261201
TABLE_POSITIONS = 4097
SAMPLED_POSITIONS = sorted(set([0, 1, 2, 3, 15, 16, 17, 31, 32, 127, 128, 129, 255, 256, 1000,
                                1023, 1024, 2047, 2048, 2049, 3071, 3072, 4095, 4096]
                               + list(range(5, 4097, 97))))
# (n_q_heads, n_kv_heads, positions) of the forward() cases
DECODE_CASES = [(8, 2, [0, 1, 5, 16, 127, 128, 129, 200]), (64, 8, [0, 3, 130])]


def bf16_bits(rng, shape, scale=1.0):
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)  # truncation: any bf16 value will do


def main() -> None:
    if not O.ref_available():
        raise SystemExit("oracle/_ref/libref.so is missing: run oracle/build_ref.sh first")
    rng = np.random.default_rng(SEED)
    out: dict[str, np.ndarray] = {}

    # RoPE table: sampled rows, and a digest of the whole [0, 4096] table.
    full = np.stack([np.concatenate(O.ref_cos_sin(p)) for p in range(TABLE_POSITIONS)])
    out["table_positions"] = np.array(SAMPLED_POSITIONS, np.int32)
    out["table_cos"] = full[SAMPLED_POSITIONS, :32].copy()
    out["table_sin"] = full[SAMPLED_POSITIONS, 32:].copy()
    h = hashlib.sha256(np.ascontiguousarray(full[:, :32]).tobytes()
                       + np.ascontiguousarray(full[:, 32:]).tobytes()).hexdigest()
    out["table_sha256"] = np.frombuffer(h.encode(), np.uint8)

    # apply_rotary_emb on random heads at a few positions.
    rot_pos = np.array([0, 1, 77, 1000, 4096], np.int32)
    rot_in = (rng.standard_normal((len(rot_pos), 4, 64)) * 3).astype(np.float32)
    rot_out = np.stack([O.ref_rotate(rot_in[i].reshape(-1), full[p, :32], full[p, 32:])
                        .reshape(4, 64) for i, p in enumerate(rot_pos)])
    out["rot_pos"], out["rot_in"], out["rot_out"] = rot_pos, rot_in, rot_out

    # softmax, including a -inf entry and a large spread.
    sm_in = (rng.standard_normal((6, 33)) * np.array([1, 5, 20, 50, 0.1, 3])[:, None]
             ).astype(np.float32)
    sm_in[2, 7] = -np.inf
    out["softmax_in"] = sm_in
    out["softmax_out"] = np.stack([O.ref_softmax(r) for r in sm_in])

    # forward() decode cases.
    idx = 0
    for hq, hkv, positions in DECODE_CASES:
        d = 64
        for pos in positions:
            # One input set per position, run through a full and a window layer.
            row = (rng.standard_normal((hq + 2 * hkv) * d) * 0.8).astype(np.float32)
            kh = bf16_bits(rng, (pos, hkv * d))
            vh = bf16_bits(rng, (pos, hkv * d))
            sinks = rng.standard_normal(hq).astype(np.float32)
            p = f"case{idx}_"
            out[p + "meta"] = np.array([hq, hkv, pos, 128], np.int32)
            out[p + "qkv"] = row
            out[p + "k_hist_bf16"] = kh
            out[p + "v_hist_bf16"] = vh
            out[p + "sinks"] = sinks
            for window_layer in (False, True):
                o, k_rot = O.ref_decode_one(row, O.from_bf16(kh), O.from_bf16(vh), sinks, pos,
                                            hq, hkv, window=128, window_layer=window_layer)
                tag = "win" if window_layer else "full"
                out[p + "out_" + tag] = o
                out[p + "k_rot_" + tag] = k_rot
            idx += 1
    out["n_cases"] = np.array([idx], np.int32)
    path = os.path.join(HERE, "ref_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {idx} forward() cases)")


if __name__ == "__main__":
    main()
