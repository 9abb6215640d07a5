"""Seeded synthetic WKV7 inputs with the measurement harness's distributions.

Token distributions (per head, D features):
  r, k, v ~ N(0, 1); retention w = exp(-exp(u)), u ~ U(u_low, 0);
  kk = kappa / |kappa| with kappa ~ N(0, 1); a = -kk; b = kk * g,
  g = sigmoid(N(0, 1)).
Everything is generated in fp32 on the generator's device and then cast to
the requested io dtype; consumers (kernels and the oracle) read the cast
values. Packed layout is [N, H, D]; pools are [slots, H, D, D] ([K,V]).
"""

from __future__ import annotations

import math

import torch

EXP_NEG_HALF = math.exp(-0.5)
# Smallest / largest retention reachable through decay logits.
LOGITS_W_MIN = math.exp(-EXP_NEG_HALF)


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def make_tokens(n_tokens: int, heads: int, head_size: int, *, dtype: torch.dtype,
                seed: int, device="cpu", u_low: float = -5.0) -> dict[str, torch.Tensor]:
    """Returns r, w (retention), k, v, a, b as contiguous [N, H, D] tensors."""
    g = _gen(seed, device)
    shape = (n_tokens, heads, head_size)

    def randn():
        return torch.randn(shape, generator=g, device=device, dtype=torch.float32)

    r = randn()
    k = randn()
    v = randn()
    u = torch.rand(shape, generator=g, device=device, dtype=torch.float32) * (-u_low) + u_low
    w = torch.exp(-torch.exp(u))
    kk = randn()
    kk = kk / kk.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    gate = torch.sigmoid(randn())
    a = -kk
    b = kk * gate
    out = {"r": r, "w": w, "k": k, "v": v, "a": a, "b": b}
    return {name: t.to(dtype).contiguous() for name, t in out.items()}


def logits_from_retention(w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Decay logits x with exp(-e^{-1/2} sigmoid(x)) == w, for representable w.

    w below exp(-e^{-1/2}) (about 0.5453) is not reachable through logits;
    such entries are clamped to the floor.
    """
    sig = (-torch.log(w.float()) / EXP_NEG_HALF).clamp(eps, 1.0 - eps)
    return torch.log(sig) - torch.log1p(-sig)


def make_case(*, lengths, heads: int, head_size: int, dtype: torch.dtype, seed: int,
              state_std: float = 0.1, pool_slots: int | None = None, slots=None,
              u_low: float = -5.0, device="cpu") -> dict:
    """A packed varlen case: tokens, cu_seqlens, state_indices and an fp32 pool."""
    lengths = [int(x) for x in lengths]
    total = sum(lengths)
    tokens = make_tokens(total, heads, head_size, dtype=dtype, seed=seed,
                         device=device, u_low=u_low)
    offsets = [0]
    for length in lengths:
        offsets.append(offsets[-1] + length)
    if pool_slots is None:
        pool_slots = len(lengths)
    if slots is None:
        slots = list(range(len(lengths)))
    g = _gen(seed + 1, device)
    pool = torch.randn((pool_slots, heads, head_size, head_size), generator=g,
                       device=device, dtype=torch.float32) * state_std
    case = dict(tokens)
    case["cu_seqlens"] = torch.tensor(offsets, dtype=torch.int32, device=device)
    case["state_indices"] = torch.tensor(list(slots), dtype=torch.int32, device=device)
    case["state_pool"] = pool.contiguous()
    return case


def varlen_lengths(count: int = 64, low: int = 128, high: int = 4096,
                   seed: int = 20260807) -> list[int]:
    """Sequence lengths uniform in [low, high] (seeded, CPU). The defaults are
    benchmark config 3's varlen batch: 64 sequences, lengths in [128, 4096]."""
    g = _gen(seed, "cpu")
    return [int(x) for x in torch.randint(low, high + 1, (count,), generator=g)]

