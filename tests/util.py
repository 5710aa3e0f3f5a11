"""Input generators shared by the tests (not a checker: inputs only)."""
import numpy as np

from oracle import row_bytes, Q8_0, Q5_0, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS

BLOCK_BYTES = {Q8_0: 34, Q5_0: 22, Q4_K: 144, Q6_K: 210, IQ2_XXS: 66, IQ3_XXS: 98}


def sane_rows(fmt, rows, cols, rng):
    """Random block bytes with finite fp16 scales, the reference tests' recipe
    (tests/test_quants.cpp:109-128, tests/test_runtime.cpp:477-487)."""
    w = rng.integers(0, 256, size=rows * row_bytes(fmt, cols), dtype=np.uint8)
    blocks = w.reshape(-1, BLOCK_BYTES[fmt])
    def half():
        return (0x2000 | (rng.integers(0, 1 << 16, size=blocks.shape[0]) & 0x0BFF)).astype(np.uint16)
    if fmt == Q6_K:
        blocks[:, 208:210] = half().view(np.uint8).reshape(-1, 2)
    else:
        blocks[:, 0:2] = half().view(np.uint8).reshape(-1, 2)
        if fmt == Q4_K:
            blocks[:, 2:4] = half().view(np.uint8).reshape(-1, 2)
    return w


def normal_weights(rows, cols, rng, std=0.02):
    return (rng.standard_normal((rows, cols)) * std).astype(np.float32)


def activations(nx, cols, rng, outliers=False):
    x = rng.standard_normal((nx, cols)).astype(np.float32)
    if outliers:
        x[rng.random(x.shape) < 0.01] *= 20.0
    return x


class tuned:
    """Development tuning overrides for one block: sets the FLH_* variables,
    re-reads them into the library (flh_init re-reads the environment), and
    restores both afterwards."""

    def __init__(self, flh, **env):
        self.flh, self.env = flh, env

    def __enter__(self):
        import os
        self.old = {k: os.environ.get(k) for k in self.env}
        os.environ.update({k: str(v) for k, v in self.env.items()})
        self.flh.init(0)
        return self

    def __exit__(self, *exc):
        import os
        for k, v in self.old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
        self.flh.init(0)
        return False
