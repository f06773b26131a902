"""Writes the committed golden fixtures of this directory (run from the repo root:
``python tests/golden/make_golden.py``).

* ``hadamard_signs_h40_d128_seed0.npy`` -- the random Q/K Hadamard signs of the
  reference (hadamard.py:58-62): ``torch.Generator("cpu").manual_seed(0)``,
  ``randint(0, 2, (40, 128), int8) * 2 - 1``.  Pins the sign stream the oracle
  and the product use (H=40, D=128 is the Wan2.1-14B head layout) against
  changes of torch's CPU generator.
* ``e4m3_bf16_codes.npy`` -- uint8[65536]: entry i is the E4M3FN code that
  ``torch.float8_e4m3fn`` gives for the bf16 value with bit pattern i, clamped
  to [-448, 448] first as every quantiser of the reference does
  (quant_triton.py:49-57; Triton's ``float8e4nv`` is the same format);
  non-finite patterns hold 0x7F.
"""
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def main() -> None:
    gen = torch.Generator(device="cpu").manual_seed(0)
    s = torch.randint(0, 2, (40, 128), generator=gen, dtype=torch.int8).mul_(2).sub_(1)
    np.save(os.path.join(HERE, "hadamard_signs_h40_d128_seed0.npy"), s.numpy())
    vals = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    finite = np.isfinite(vals)
    x = np.clip(np.where(finite, vals, 0.0), -448.0, 448.0).astype(np.float32)
    codes = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    codes = np.where(finite, codes, 0x7F).astype(np.uint8)
    np.save(os.path.join(HERE, "e4m3_bf16_codes.npy"), codes)


if __name__ == "__main__":
    main()
