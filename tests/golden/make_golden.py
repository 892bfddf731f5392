"""Writes tests/golden/codecs.npz: codec golden vectors from torch's own
float8/bfloat16 conversions (independent library routines, not the
reference). Run from the repo root: python tests/golden/make_golden.py

Contents:
  e4m3_all      float32[256]  value of every E4M3FN byte (torch float8_e4m3fn)
  e8m0_all      float32[256]  value of every E8M0 byte (torch float8_e8m0fnu)
  enc_x         float32[N]    inputs in [-448, 448] incl. every exact midpoint
  enc_e4m3      uint8[N]      torch RNE float32 -> float8_e4m3fn bytes
  bf16_x        float32[M]    random fp32 incl. bf16 midpoints
  bf16_bits     uint16[M]     torch RNE float32 -> bfloat16 bits
"""
import os

import numpy as np
import torch


def main():
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "codecs.npz")
    u8 = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    e4m3_all = u8.view(torch.float8_e4m3fn).to(torch.float32).numpy()
    e8m0_all = u8.view(torch.float8_e8m0fnu).to(torch.float32).numpy()
    rng = np.random.default_rng(1234)
    xs = [rng.standard_normal(4096).astype(np.float32) * s
          for s in (1e-3, 2e-2, 0.3, 3.0, 60.0)]
    fin = e4m3_all[:0x7F].astype(np.float64)
    mids = ((fin[1:] + fin[:-1]) / 2).astype(np.float32)
    x = np.concatenate(xs + [mids, -mids, e4m3_all[:0x7F], -e4m3_all[1:0x7F]])
    x = np.clip(x, -448, 448).astype(np.float32)
    enc = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    b = rng.standard_normal(8192).astype(np.float32) * 10
    bits = b.view(np.uint32)
    mid = ((bits & 0xFFFF0000) | 0x8000).view(np.float32)[:2048]
    bx = np.concatenate([b, mid]).astype(np.float32)
    bbits = torch.from_numpy(bx).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.savez_compressed(out, e4m3_all=e4m3_all, e8m0_all=e8m0_all, enc_x=x,
                        enc_e4m3=enc, bf16_x=bx, bf16_bits=bbits)
    print("wrote", out, x.size, bx.size)


if __name__ == "__main__":
    main()
