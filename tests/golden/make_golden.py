"""Writes the golden fixtures of this directory from the CPU oracle (oracle/pa_oracle.c):

    python tests/golden/make_golden.py

  attn_cases.npz    small partial-attention cases: K, V rows (q8_0 / q4_0 / f16), Q, and the oracle's outputs - the
                    ggml-faithful restatement (orc_attn_ggml: Q -> q8_0 blocks, int block dots, online softmax) and the
                    fp64 closed form with the reference engines' rounding (orc_attn_exact, Q -> f16(q*scale)).
                    Cases cover the decode kernel's shape (8 rows, even KV heads, head dim 128), the general kernel
                    (16 / 12 rows, head dim 256), ragged key counts, padded rows and an empty call.
  quant_cases.npz   ggml-semantics q8_0 / q4_0 blocks of edge-value rows (zeros, ties at .5, +-max, tiny, huge).
  accept_cases.npz  greedy acceptance over logits [17][1031] with planted draft prefixes and exact ties.

The fixtures pin the oracle against later edits (tests/test_golden.py) and let the GPU tests check the HIP path against
stored answers (tests/test_gpu_golden.py). Everything is seeded; rerunning reproduces the files byte for byte on the
same oracle build.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
import oracle as orc  # noqa: E402

# (name, fmt, nkv, rows, hd, n_keys, row padding bytes, seed, K outlier channels)
ATTN_CASES = [
    ("q8_decode", orc.Q8_0, 2, 8, 128, 77, 0, 11, 2),
    ("q4_decode", orc.Q4_0, 2, 8, 128, 100, 0, 12, 0),
    ("q8_decode_3rows", orc.Q8_0, 4, 3, 128, 33, 0, 13, 0),
    ("q8_verify", orc.Q8_0, 1, 16, 128, 130, 0, 14, 0),
    ("q8_hd256_padded", orc.Q8_0, 2, 12, 256, 65, 48, 15, 0),
    ("f16_decode", orc.F16, 2, 8, 128, 40, 0, 16, 0),
    ("q8_empty", orc.Q8_0, 2, 8, 128, 0, 0, 17, 0),
]


def attn_cases():
    out = {}
    names = []
    for name, fmt, nkv, rows, hd, nk, pad, seed, outl in ATTN_CASES:
        hb = orc.head_bytes(fmt, hd)
        rs = nkv * hb + pad
        K = orc.fill_rows(seed, fmt, nkv, hd, nk, rs=rs, n_outliers=outl, outlier_mul=8.0)
        V = orc.fill_rows(seed + 1000, fmt, nkv, hd, nk, rs=rs)
        Q = orc.normal(seed + 2000, 0, nkv * rows * hd).reshape(nkv * rows, hd)
        meta = np.array([fmt, nkv, rows, hd, nk, rs], np.int64)
        sg = orc.make_shape(nkv, rows, hd, fmt, orc.QMODE_GGML, rs=rs)
        Og, mg, lg = orc.attn_ggml(sg, Q, K, V, nk, 1)
        se = orc.make_shape(nkv, rows, hd, fmt, orc.QMODE_F16, rs=rs)
        Oe, me, le = orc.attn_exact(se, Q, K, V, nk, 1)
        for k, v in (("meta", meta), ("K", K), ("V", V), ("Q", Q), ("O_ggml", Og), ("m_ggml", mg), ("l_ggml", lg),
                     ("O_exact_f16q", Oe), ("m_exact_f16q", me), ("l_exact_f16q", le)):
            out[f"{name}__{k}"] = v
        names.append(name)
    out["names"] = np.array(names)
    return out


def quant_cases():
    rng = np.random.default_rng(5)
    x = np.zeros((8, 64), np.float32)
    x[1, :] = (np.arange(64) - 32) * 0.5                      # ties at .5 after scaling
    x[2, :] = rng.standard_normal(64).astype(np.float32)
    x[3, :32] = 127.0; x[3, 32:] = -127.0
    x[4, :] = 1e-30                                            # d underflows to a subnormal fp16 / zero
    x[5, :] = rng.standard_normal(64).astype(np.float32) * 1e4
    x[6, ::2] = -8.0; x[6, 1::2] = 7.0
    x[7, :] = rng.uniform(-1, 1, 64).astype(np.float32); x[7, 17] = -3.0   # q4_0: the signed max is negative
    flat = x.reshape(-1)
    return {"x": x, "q8_0": orc.quantize(orc.Q8_0, flat), "q4_0": orc.quantize(orc.Q4_0, flat)}


def accept_cases():
    rng = np.random.default_rng(9)
    vocab, n_rows = 1031, 17
    cases = {}
    for c, k_true in enumerate((0, 5, 16)):
        logits = rng.standard_normal((n_rows, vocab)).astype(np.float32)
        draft = rng.integers(0, vocab, n_rows - 1).astype(np.int32)
        for i in range(min(k_true, n_rows - 1)):
            logits[i, draft[i]] = logits[i].max() + 0.25
            j = int(rng.integers(0, vocab))                    # an exact tie: the lower index wins
            logits[i, j] = logits[i, draft[i]]
            if j < draft[i]:
                draft[i] = j
        if k_true < n_rows - 1 and np.argmax(logits[k_true]) == draft[k_true]:
            logits[k_true, draft[k_true]] = logits[k_true].min() - 1.0
        k, bonus, am = orc.accept(logits, draft)
        cases[f"c{c}_logits"] = logits
        cases[f"c{c}_draft"] = draft
        cases[f"c{c}_expect"] = np.concatenate([[k, bonus], am]).astype(np.int32)
    return cases


def main():
    np.savez_compressed(HERE / "attn_cases.npz", **attn_cases())
    np.savez_compressed(HERE / "quant_cases.npz", **quant_cases())
    np.savez_compressed(HERE / "accept_cases.npz", **accept_cases())
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
