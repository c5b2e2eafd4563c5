"""Synthetic 3x800x800 input pages for PP-DocLayoutV3 (CHW float32 in [0, 1],
the layout ppdl_infer takes): the benchmark and test workloads.

document_page: a page-like image (background, text lines, blocks, rules).
uniform_page:  seeded U(0,1) pixels, the full-network benchmark input.
"""
import numpy as np

PAGE = 800


def uniform_page(seed=0):
    """3 x 800 x 800 i.i.d. U(0,1) float32 from numpy's seeded PCG64."""
    return np.random.default_rng(seed).random((3, PAGE, PAGE), dtype=np.float32)


def document_page(seed=0):
    """A synthetic page (3, 800, 800) in [0, 1]: light background, dark text
    lines, a few filled blocks (figures/tables) and rules."""
    rng = np.random.default_rng(seed)
    img = np.full((3, PAGE, PAGE), 0.96, np.float32)
    img += rng.normal(0, 0.01, img.shape).astype(np.float32)
    y = 40
    while y < PAGE - 60:
        kind = rng.random()
        if kind < 0.2:  # figure / table block
            h = int(rng.integers(80, 200))
            x0, x1 = int(rng.integers(40, 200)), int(rng.integers(500, 760))
            img[:, y:y + h, x0:x1] = rng.uniform(0.2, 0.8, (3, 1, 1)).astype(np.float32)
            y += h + 20
        elif kind < 0.3:  # title
            img[:, y:y + 18, 60:int(rng.integers(250, 500))] = 0.1
            y += 40
        else:  # paragraph of text lines
            for _ in range(int(rng.integers(2, 7))):
                x = 60
                while x < 740:
                    wlen = int(rng.integers(10, 60))
                    img[:, y:y + 8, x:min(x + wlen, 740)] = 0.15
                    x += wlen + 8
                y += 14
            y += 16
    return np.clip(img, 0.0, 1.0).astype(np.float32)
