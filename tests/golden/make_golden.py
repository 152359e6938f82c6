"""Write tests/golden/sdpa_cases.npz: small decode / prefill cases whose expected outputs come from
an implementation independent of the oracle -- torch's float64 CPU scaled_dot_product_attention
(GQA 16:2 via enable_gqa, scale 1/sqrt(256), causal mask offset by pos0) times the sigmoid gate.

Inputs are drawn with the oracle's portable generator; the fixture stores the expected outputs and
a SHA-256 of the input bytes, so a test regenerates the inputs, checks the digest (pinning the
generator) and compares the oracle's outputs with torch's (pinning head grouping, scale, causal
offset and gate address).

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent / "sdpa_cases.npz"
H, KV, D = 16, 2, 256


def sdpa(q, k, v, gate, pos0):
    """q [T][16][256] f32, k/v [2][S][256] f32 (f16 values), gate [T][16][256]; causal, token t
    sees keys [0, pos0 + t]."""
    T, S = q.shape[0], k.shape[1]
    qt = torch.from_numpy(q.astype(np.float64)).permute(1, 0, 2)[None]   # [1,16,T,256]
    kt = torch.from_numpy(k.astype(np.float64))[None]                    # [1,2,S,256]
    vt = torch.from_numpy(v.astype(np.float64))[None]
    mask = torch.arange(S)[None, :] <= (pos0 + torch.arange(T))[:, None]  # [T,S]
    o = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, enable_gqa=True)
    o = o[0].permute(1, 0, 2).numpy()                                    # [T,16,256]
    return o / (1.0 + np.exp(-gate.astype(np.float64)))


def digest(*arrays) -> np.ndarray:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return np.frombuffer(h.digest(), dtype=np.uint8).copy()


def main():
    cases = {}
    # Decode: len keys, the single query at position len - 1 (sees all keys).
    for length, scale in ((1, 1.0), (7, 2.0), (33, 1.0)):
        d = O.decode_inputs(5000 + length, length, length + 3, q_scale=scale)
        max_ctx = d["max_ctx"]
        k = O.f16_to_f32(d["k"]).reshape(KV, max_ctx, D)[:, :length]
        v = O.f16_to_f32(d["v"]).reshape(KV, max_ctx, D)[:, :length]
        q = d["q"].reshape(1, H, D)
        gate = d["qg"].reshape(H, 2 * D)[:, D:][None]
        exp = sdpa(q, k, v, gate, length - 1)[0]
        tag = f"decode_{length}"
        cases[tag + "_sha256"] = digest(d["q"], d["qg"], d["k"], d["v"])
        cases[tag + "_meta"] = np.array([5000 + length, length, max_ctx, int(scale)], np.int64)
        cases[tag + "_out"] = exp
    # Prefill: n tokens after pos0 cached keys.
    for pos0, n in ((0, 5), (9, 4), (31, 3)):
        p = O.prefill_inputs(6000 + 17 * pos0 + n, pos0, n, pos0 + n + 2, q_scale=2.0)
        max_ctx = p["max_ctx"]
        k = O.f16_to_f32(p["k"]).reshape(KV, max_ctx, D)[:, :pos0 + n]
        v = O.f16_to_f32(p["v"]).reshape(KV, max_ctx, D)[:, :pos0 + n]
        q = p["q"].reshape(n, H, D)
        gate = p["qg"].reshape(n, H, 2 * D)[:, :, D:]
        exp = sdpa(q, k, v, gate, pos0)
        tag = f"prefill_{pos0}_{n}"
        cases[tag + "_sha256"] = digest(p["q"], p["qg"], p["k"], p["v"])
        cases[tag + "_meta"] = np.array([6000 + 17 * pos0 + n, pos0, n, max_ctx], np.int64)
        cases[tag + "_out"] = exp
    # Generator pins: first values of each stream used above.
    cases["gen_normal_seed7"] = O.normal(7, 16)
    cases["gen_normal_f16_seed7"] = O.normal_f16(7, 16)
    np.savez_compressed(OUT, **cases)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(cases)} arrays)")


if __name__ == "__main__":
    main()
