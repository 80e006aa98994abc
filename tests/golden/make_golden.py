"""Writes the golden fixtures in this directory from the (pinned) CPU oracle.

    python tests/golden/make_golden.py

Each fixture holds seeded inputs and the oracle's outputs for them, small
enough to commit.  The reference itself holds no golden tensors for this path
(its tests compare end-to-end text), so these are this build's own vectors:
the oracle that produced them is pinned by tests/test_oracle_pinning.py and
tests/test_oracle_reference.py.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

import oracle  # noqa: E402
from oracle import reference as R  # noqa: E402


def quant_fixture(wtype: str, rows: int, k: int, seed: int) -> dict:
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, k)) * 0.02).astype(np.float32)
    w[0] = 0.0                                    # special rows ride along
    w[1] = -0.75
    packed = getattr(oracle, f"quantize_{wtype}")(w)
    deq = getattr(oracle, f"dequant_{wtype}")(packed, k)
    x = R.bf16_round(rng.standard_normal(k).astype(np.float32))
    y = R.gemv_ref(x, deq)
    return {"w": w, "packed": packed, "x_bf16": x, "y_ref": y}


def attention_fixture(seed: int) -> dict:
    rng = np.random.default_rng(seed)
    nh, nk, d, s_cap, pos = 8, 2, 128, 200, 150
    kc = R.bf16_round(rng.standard_normal((s_cap, nk, d)).astype(np.float32))
    vc = R.bf16_round(rng.standard_normal((s_cap, nk, d)).astype(np.float32))
    q = (rng.standard_normal((nh, d)) * 2).astype(np.float32)
    kn = (rng.standard_normal((nk, d)) * 2).astype(np.float32)
    vn = rng.standard_normal((nk, d)).astype(np.float32)
    qw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    cos, sin = R.rope_cos_sin(np.array([pos]), d, 1e6)
    qr = R.qk_norm_rope(q, qw, cos, sin)
    kr = R.qk_norm_rope(kn, kw, cos, sin)
    kref, vref = kc.copy(), vc.copy()
    kref[pos] = R.bf16_round(kr.astype(np.float32))
    vref[pos] = R.bf16_round(vn)
    out = R.attention_ref(qr[None], kref[:pos + 1], vref[:pos + 1])[0]
    return {"k_cache": kc, "v_cache": vc, "q": q, "k_new": kn, "v_new": vn, "q_norm": qw, "k_norm": kw,
            "pos": np.int32(pos), "theta": np.float64(1e6), "out_ref": out}


FIXTURES = {
    "q4_k_k1024.npz": lambda: quant_fixture("q4_k", 24, 1024, 101),
    "q6_k_k512.npz": lambda: quant_fixture("q6_k", 16, 512, 102),
    "q8_0_k256.npz": lambda: quant_fixture("q8_0", 16, 256, 103),
    "attn_decode_gqa4.npz": lambda: attention_fixture(104),
}


def main() -> None:
    for name, make in FIXTURES.items():
        np.savez_compressed(HERE / name, **make())
        print(f"wrote {name} ({(HERE / name).stat().st_size} bytes)")


if __name__ == "__main__":
    main()
