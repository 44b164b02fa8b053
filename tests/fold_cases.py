"""Adversarial rows for the sequential-sum fold (nd_fold_rows).

Every generator returns float32 rows [rows, n].  The truth for a row is its
sequential float32 sum ((0 + x0) + x1) + ..., which numpy's add.accumulate
computes element by element (tests/test_fold_cpu.py checks that against a
Python loop)."""
import numpy as np

SCALES = (1.0, 1e-3, 1e3, 1e-20, 2.0 ** -140)


def _bits(u):
    return np.asarray(u, dtype=np.uint32).view(np.float32)


def rows_of(kind, rows, n, rng):
    if kind == "squares":
        out = []
        for r in range(rows):
            g = rng.standard_normal(n).astype(np.float32) * np.float32(SCALES[r % len(SCALES)])
            out.append(g * g)
        return np.stack(out)
    if kind == "exps":
        return np.exp(rng.standard_normal((rows, n)).astype(np.float32) * np.float32(3.0)
                      - np.float32(6.0)).astype(np.float32)
    if kind == "few_bits":  # frequent exact ties
        m = rng.integers(1, 16, (rows, n)).astype(np.float32)
        return np.ldexp(m, rng.integers(-20, 20, (rows, n))).astype(np.float32)
    if kind == "zeros":
        g = rng.standard_normal((rows, n)).astype(np.float32)
        x = g * g
        x[:, : n // 3] = 0.0
        x[rng.random((rows, n)) < 0.25] = 0.0
        return x
    if kind == "subnormal":
        return _bits(rng.integers(0, 0x01800000, (rows, n)))
    if kind == "pow2":
        return np.ldexp(np.ones((rows, n), np.float32), rng.integers(-12, 12, (rows, n))).astype(np.float32)
    if kind == "crossing":  # each term about the running sum
        x = np.empty((rows, n), np.float32)
        s = np.full(rows, 1e-3)
        for i in range(n):
            t = s * (0.5 + rng.random(rows))
            x[:, i] = t
            s = np.where(s + t > 1e30, 1e-3, s + t)
        return x
    if kind == "one_large":
        g = rng.standard_normal((rows, n)).astype(np.float32)
        x = g * g
        x[:, n // 7] = 1e8
        return x
    if kind == "bit_patterns":
        return _bits(rng.integers(0, 0x6F000000, (rows, n)))
    if kind == "uniform24":
        return (rng.integers(0, 1 << 24, (rows, n)).astype(np.float32) * np.float32(2.0 ** -24))
    if kind == "signed":  # not the parallel path: negatives and -0 among the terms
        x = rng.standard_normal((rows, n)).astype(np.float32)
        x[rng.random((rows, n)) < 0.05] = -0.0
        return x
    if kind == "inf":
        g = rng.standard_normal((rows, n)).astype(np.float32)
        x = g * g
        x[:, n // 2] = np.inf
        return x
    raise ValueError(kind)


KINDS = ("squares", "exps", "few_bits", "zeros", "subnormal", "pow2", "crossing", "one_large",
         "bit_patterns", "uniform24", "signed", "inf")


def sequential_sums(x):
    """((0 + x[r,0]) + x[r,1]) + ... in float32, per row."""
    x = np.asarray(x, dtype=np.float32)
    acc = np.add.accumulate(np.concatenate([np.zeros((x.shape[0], 1), np.float32), x], axis=1),
                            axis=1, dtype=np.float32)
    return acc[:, -1]
