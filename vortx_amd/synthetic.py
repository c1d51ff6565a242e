"""Seeded synthetic operands of the benchmark configurations (torch, any device).

Quantized weights follow the value distributions of the measured configs:
  Q8_0  q ~ U{-127..127}, d = f16(|N(0, 0.02)| * max|q| / 127) per block
  Q4_0  nibbles ~ U{0..15}, d = f16(|N(0, 0.02)| / 8)
  Q4_K  nibbles ~ U{0..15}, the 12 packed scale bytes uniform (so every 6-bit
        scale and min is uniform in 0..63), d, dmin = f16(|N(0, 0.01)|)
Activations x ~ N(0, 1) stored [B, K]; dense GEMM operands ~ U[-1, 1].
"""
from __future__ import annotations

import torch

QTYPE_INFO = {2: (32, 18), 8: (32, 34), 12: (256, 144)}


def row_bytes(qtype: int, K: int) -> int:
    qk, bb = QTYPE_INFO[qtype]
    if K % qk:
        raise ValueError(f"K={K} is not a multiple of {qk}")
    return K // qk * bb


def _f16_bytes(v: torch.Tensor) -> torch.Tensor:
    """[..., n] float -> [..., n, 2] uint8 (little-endian binary16)."""
    h = v.to(torch.float16).contiguous()
    return h.view(torch.uint8).reshape(*h.shape, 2)


def quant_weights(qtype: int, M: int, K: int, seed: int, device="cpu") -> torch.Tensor:
    """uint8 tensor [M, row_bytes] of random blocks of `qtype`."""
    qk, bb = QTYPE_INFO[qtype]
    nb = K // qk
    if K % qk:
        raise ValueError(f"K={K} is not a multiple of {qk}")
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    blocks = torch.randint(0, 256, (M, nb, bb), dtype=torch.uint8, generator=g, device=device)
    if qtype == 8:
        qs = torch.randint(-127, 128, (M, nb, 32), dtype=torch.int16, generator=g, device=device)
        amax = qs.abs().amax(-1).to(torch.float32)
        z = torch.randn((M, nb), generator=g, device=device) * 0.02
        blocks[..., 0:2] = _f16_bytes(z.abs() * amax / 127.0)
        blocks[..., 2:] = qs.to(torch.int8).view(torch.uint8)
    elif qtype == 2:
        z = torch.randn((M, nb), generator=g, device=device) * 0.02
        blocks[..., 0:2] = _f16_bytes(z.abs() / 8.0)
    elif qtype == 12:
        z = torch.randn((M, nb, 2), generator=g, device=device) * 0.01
        blocks[..., 0:4] = _f16_bytes(z.abs()).reshape(M, nb, 4)
    else:
        raise ValueError(f"unknown qtype {qtype}")
    return blocks.reshape(M, nb * bb)


def activations(B: int, K: int, seed: int, device="cpu") -> torch.Tensor:
    """x ~ N(0, 1), stored [B, K] contiguous (the [K, B] operand is its transpose)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.randn((B, K), generator=g, device=device, dtype=torch.float32)


def uniform(shape, seed: int, device="cpu") -> torch.Tensor:
    """i.i.d. U[-1, 1] f32."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.rand(shape, generator=g, device=device, dtype=torch.float32) * 2.0 - 1.0
