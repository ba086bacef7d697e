"""Shared input generation for the tests (CPU generator: identical on every host)."""
import numpy as np
import torch

E = 64


def bits16(t):
    """16-bit tensor -> its uint16 bit pattern as numpy."""
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits16(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype)


def make_inputs(seed, B, H, L, D=64, dtype=torch.bfloat16, rms_qk=False, tan_scale=0.1,
                tangent=True):
    """q,k,v (and dq,dk,dv) drawn from a CPU generator, cast to `dtype`.

    rms_qk: per-token RMS-normalise q and k in fp32 before the cast (Config 2).
    """
    g = torch.Generator().manual_seed(seed)
    x = [torch.randn(B, H, L, D, generator=g) for _ in range(3)]
    if rms_qk:
        for i in (0, 1):
            x[i] = x[i] * torch.rsqrt(x[i].pow(2).mean(-1, keepdim=True) + 1e-6)
    out = [t.to(dtype) for t in x]
    if tangent:
        out += [(torch.randn(B, H, L, D, generator=g) * tan_scale).to(dtype) for _ in range(3)]
    return out


def rel_l2(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def max_abs(a, b):
    return (a.double() - b.double()).abs().max().item()
