"""Seeded synthetic inputs shared by the tests (numpy, host side)."""
import numpy as np


def kv_f16(rng, n_tok, num_kv, hd, outlier_frac=0.02, outlier_scale=8.0):
    """fp16 K or V rows [n_tok][num_kv][hd] ~ N(0,1), with round(frac*hd)
    fixed outlier channels per head scaled by outlier_scale (the same channels
    for every token, as in the reference's fixed-channel outlier regime)."""
    x = rng.standard_normal((n_tok, num_kv, hd)).astype(np.float32)
    n_out = int(round(outlier_frac * hd))
    if n_out:
        for h in range(num_kv):
            ch = rng.choice(hd, n_out, replace=False)
            x[:, h, ch] *= outlier_scale
    return x.astype(np.float16)


def q_f16(rng, sub_n, num_q, hd):
    return rng.standard_normal((sub_n, num_q, hd)).astype(np.float16)


def rel_err(out, ref):
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(out - ref)) / (den if den > 0 else 1.0))
