"""Fit the router bias of the large imbalanced prefill workload and freeze it.

Workload: T=16384, d=2048, E=64, top-4, router weights N(0, 0.02) from the
synthetic generator (seed 5, stream 1).  The bias b[E] is added to the
logits after the product (mat_mul_add form); it is fitted on HELD-OUT tokens
(seed 1234) so that expert popularity follows Zipf(s=1.1) over the expert
index, capped at 10x the mean load: with top-4 of 64 an expert can hold at
most one slot per token, i.e. 16x the mean, and an uncapped Zipf(1.1) head
(16.5x) is infeasible.  The cap is water-filled: loads above it are clipped
and the excess is spread proportionally over the rest.

Writes zipf_bias_e64_k4.npy (64 float32) next to this script.
Run: python tests/golden/make_zipf_bias.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import orc  # noqa: E402

T_FIT, d, E, k = 8192, 2048, 64, 4
CAP = 10.0


def zipf_targets(E, k, s=1.1, cap=CAP):
    p = (np.arange(1, E + 1, dtype=np.float64)) ** (-s)
    p /= p.sum()
    mean = 1.0 / E
    for _ in range(100):
        over = p > cap * mean
        if not over.any():
            break
        excess = (p[over] - cap * mean).sum()
        p[over] = cap * mean
        p[~over] += excess * p[~over] / p[~over].sum()
    return p            # share of the T*k slots per expert


def topk_counts(logits, bias):
    z = logits + bias[None, :]
    idx = np.argpartition(-z, k - 1, axis=1)[:, :k]
    return np.bincount(idx.ravel(), minlength=E)


def main():
    wr = orc.synth((d, E), 5, 1, 0.02)
    x = orc.synth((T_FIT, d), 1234, 0, 1.0)
    logits = orc.router_logits(x, wr).astype(np.float64)
    target = zipf_targets(E, k) * T_FIT * k
    b = np.zeros(E)
    for it in range(3000):
        c = topk_counts(logits, b)
        err = np.log(target + 1.0) - np.log(c + 1.0)
        b += 0.05 * err
        b -= b.mean()
    c = topk_counts(logits, b)
    b32 = b.astype(np.float32)
    # Check on the benchmark's own tokens (seed 5) with the exact oracle route.
    xb = orc.synth((4096, d), 5, 0, 1.0)
    _, ids, _ = orc.route(xb, wr, k, b32)
    cb = np.bincount(ids.ravel(), minlength=E)
    print("fit  max/mean %.2f  top5 %s" % (c.max() / c.mean(), np.sort(c)[::-1][:5]))
    print("check max/mean %.2f (first 4096 benchmark tokens)" % (cb.max() / cb.mean()))
    np.save(os.path.join(HERE, "zipf_bias_e64_k4.npy"), b32)


if __name__ == "__main__":
    main()
