"""Writes the committed fixtures under tests/golden/ (run from the repo root).

rotation_d128_seed42.npy: the rotation of the reference's rotated backend,
Q of torch.linalg.qr(torch.randn(128, 128, generator=CPU Generator seeded 42))
(fade/rotated_quant.py:91-96), generated with torch itself.
"""

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def main() -> None:
    gen = torch.Generator().manual_seed(42)
    q, _ = torch.linalg.qr(torch.randn(128, 128, generator=gen))
    np.save(os.path.join(HERE, "rotation_d128_seed42.npy"), q.numpy().astype(np.float32))


if __name__ == "__main__":
    main()
