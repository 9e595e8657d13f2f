"""Writes the golden vectors in this directory from torch's float8_e4m3fn
cast and float64 closed forms (not from the oracle), so the oracle tests
check against an independent implementation:

  e4m3_cases.npz  x (float32), codes (uint8) = torch cast of x (no NaN cases)
  quant_kat.npz   x [256, 256] with edge blocks; q/s (1x128, scale = amax/448),
                  q_pow2/s_pow2 (scale = 2**ceil(log2(amax/448))), q_mx/c_mx
                  (1x32, e8m0 code = floor(log2(amax)) - 8 + 127)

    python tests/golden/make_golden.py
"""

import math
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent


def cast(t):
    return t.to(torch.float8_e4m3fn).view(torch.uint8)


def main():
    rng = np.random.default_rng(1234)
    vals = torch.arange(127, dtype=torch.uint8).view(torch.float8_e4m3fn).double()
    mids = (vals[1:] + vals[:-1]) / 2
    x = torch.cat([vals, -vals, mids, -mids, torch.tensor(rng.standard_normal(4000) * 50),
                   torch.tensor([463.9, 464.0, 448.0, 2 ** -10, 3 * 2 ** -11])]).float()
    np.savez(OUT / "e4m3_cases.npz", x=x.numpy(), codes=cast(x).numpy())

    a = torch.tensor(rng.standard_normal((256, 256)), dtype=torch.float32)
    a[0, :128] = 0
    a[1, :128] = 1.0
    a[2, 128:] = torch.linspace(-448, 448, 128)
    a[3, :] *= 1000
    a[4, :128] = 1e-13
    a[5, :32] = 0
    a[6, 32:64] = 2.0 ** -130
    a = a.bfloat16().float()
    blocks = a.reshape(256, 2, 128)
    amax = blocks.abs().amax(-1).clamp(min=torch.tensor(1e-12))
    s = amax / 448.0
    q = cast((blocks / s[..., None]).clamp(-448, 448)).reshape(256, 256)
    s2 = torch.tensor([[2.0 ** math.ceil(math.log2(float(v))) for v in r] for r in s], dtype=torch.float32)
    q2 = cast((blocks / s2[..., None]).clamp(-448, 448)).reshape(256, 256)
    mb = a.reshape(256, 8, 32).double()
    am = mb.abs().amax(-1)
    code = torch.zeros(256, 8, dtype=torch.int64)
    for i in range(256):
        for j in range(8):
            v = float(am[i, j])
            code[i, j] = 0 if v == 0 else min(max(math.floor(math.log2(v)) - 8 + 127, 0), 254)
    qm = cast((mb * torch.pow(2.0, 127 - code.double())[..., None]).float().clamp(-448, 448)).reshape(256, 256)
    np.savez(OUT / "quant_kat.npz", x=a.numpy(), q=q.numpy(), s=s.numpy(), q_pow2=q2.numpy(),
             s_pow2=s2.numpy(), q_mx=qm.numpy(), c_mx=code.to(torch.uint8).numpy())


if __name__ == "__main__":
    main()
