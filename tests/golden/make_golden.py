"""Writes the golden fixtures under tests/golden/ (run from the repo root).

The reference holds no golden vectors for the KV path, so the fixtures pin the
oracle against the library routine the reference's FP8 semantics are written
in: torch's CPU conversion to float8_e4m3fn (fp8_kv.py:75-77,
reshape_and_cache.py:66-77 clamp to +-448 and then convert).

  e4m3_of_bf16.bin    65536 bytes: quantize(x) at scale 1.0 for every bf16 bit
                      pattern x = 0x0000..0xFFFF, i.e.
                      x.float().clamp(-448, 448).to(float8_e4m3fn)
  e4m3_scaled.npz     float32 inputs, float32 scales and the bytes of
                      (x / s).clamp(-448, 448).to(float8_e4m3fn): RNE ties,
                      subnormals, the 448/464/480 saturation boundaries, +-0,
                      +-inf and seeded normal values at scales != 1
"""

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def bf16_table() -> np.ndarray:
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    return bits.float().clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def scaled_cases():
    g = torch.Generator().manual_seed(20251201)
    edges = []
    for m in range(8):  # every subnormal step and the smallest normals
        edges += [m * 2.0 ** -9, (m + 0.5) * 2.0 ** -9, -(m + 0.5) * 2.0 ** -9]
    for e in range(-6, 9):  # ties between neighbouring codes at each binade
        for m in range(8):
            edges.append((1 + (m + 0.5) / 8) * 2.0 ** e)
    edges += [0.0, -0.0, 448.0, -448.0, 456.0, 464.0, 464.0001, 472.0, 480.0, 1e30, -1e30,
              float("inf"), float("-inf"), 2.0 ** -10, 2.0 ** -11, 1e-45]
    x_edges = torch.tensor(edges, dtype=torch.float32)
    x_rand = torch.randn(4096, generator=g) * 30.0
    xs, ss = [], []
    for s in (1.0, 0.5, 2.0, 0.015625, 3.0, 0.0123456789, 7.77):
        xs.append(x_edges * s)  # the same edges after division by s
        ss.append(torch.full_like(x_edges, s))
        xs.append(x_rand)
        ss.append(torch.full_like(x_rand, s))
    x = torch.cat(xs)
    s = torch.cat(ss)
    q = (x / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
    return x.numpy(), s.numpy(), q.numpy()


def main():
    bf16_table().tofile(os.path.join(HERE, "e4m3_of_bf16.bin"))
    x, s, q = scaled_cases()
    np.savez(os.path.join(HERE, "e4m3_scaled.npz"), x=x, scale=s, q=q)


if __name__ == "__main__":
    main()
