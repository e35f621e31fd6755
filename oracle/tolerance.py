"""Tolerance model for comparing the GPU path with the oracle.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference output is ``bf16(y)`` where ``y`` is the fp32 result of the
un-rotate -> contract -> bias -> rotate chain. Any implementation that sums
the contraction in a different order differs from ``y`` by
``|dy| <= c * u * sum_i |x_i w_i|`` (standard dot-product forward error,
``u`` the working precision), so an elementwise "<= 1 bf16 ulp" can only
hold where ``|y|`` is not much smaller than that sum. ``check_mapped``
therefore accepts an element when its bf16 (or fp16, for fp16 pools) bit
patterns are at most one ulp apart **or** ``|out - ref| <= abs_factor * bound``, where ``bound`` is the
magnitude of the chain's summands (``magnitude_bound``), and separately
requires a normwise relative error ``max|out-ref| / max|ref| <= 1e-2``.
It also reports, and bounds by the same 1e-2, the element-wise relative
error ``|out-ref| / |ref|`` over the elements whose magnitude is at least
``1 / rel_norm`` times their near-cancellation allowance (``abs_factor *
bound``): there the allowance itself is at most 1e-2 of the value, so a
larger relative error would be a real defect rather than a legitimately
reordered sum.
"""

from __future__ import annotations

import torch

from .rope import qwen_rope


def ulp_distance(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in representable steps between equal-shape bf16 or fp16 tensors.

    Both formats are sign-magnitude 16-bit patterns whose magnitudes order as
    integers, so the distance is the difference of the signed-magnitude
    integers (+0 and -0 are 0 apart).
    """

    def ordered(x):
        i = x.contiguous().view(torch.int16).to(torch.int32)
        return torch.where(i < 0, -(i & 0x7FFF), i)

    return (ordered(a) - ordered(b)).abs()


def bf16_ulp_distance(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in representable bf16 steps between equal-shape bf16 tensors."""
    return ulp_distance(a, b)


def magnitude_bound(page: torch.Tensor, spec: dict, *, position_start: int, source_theta: float,
                    target_thetas, source_scaling=None, target_scaling=None,
                    source_head_offset: int = 0) -> torch.Tensor:
    """``[2, Lt, n, Ht, D]`` fp64 bound on the summand magnitudes of each output.

    Same chain as the map with every factor replaced by its absolute value:
    |unrotated x| . |W| + |b|, then for keys |y_j| |cos| + |y_j'| |sin|.
    """
    x = page.double()
    n, dim = x.shape[2], x.shape[4]
    half = dim // 2
    pos = torch.arange(position_start, position_start + n)
    cs, ss = qwen_rope(pos, head_dim=dim, theta=source_theta, scaling=source_scaling)
    cs, ss = cs.double()[None, :, None, :half], ss.double()[None, :, None, :half]
    k = x[0]
    k1, k2 = k[..., :half], k[..., half:]
    ka = torch.cat((k1.abs() * cs.abs() + k2.abs() * ss.abs(),
                    k2.abs() * cs.abs() + k1.abs() * ss.abs()), dim=-1)
    va = x[1].abs()
    al, ah = spec["assign_layer"], spec["assign_head"]
    lt, ht, s = al.shape
    thetas = ([target_thetas] * lt if isinstance(target_thetas, (int, float)) else list(target_thetas))
    tscal = (list(target_scaling) if isinstance(target_scaling, (list, tuple))
             else [target_scaling] * lt)
    out = torch.empty(2, lt, n, ht, dim, dtype=torch.float64)
    for l in range(lt):
        ct, st = qwen_rope(pos, head_dim=dim, theta=thetas[l], scaling=tscal[l])
        ct, st = ct.double()[:, None, :half].abs(), st.double()[:, None, :half].abs()
        for h in range(ht):
            fk = torch.cat([ka[int(al[l, h, j]), :, int(ah[l, h, j]) - source_head_offset]
                            for j in range(s)], dim=-1)
            fv = torch.cat([va[int(al[l, h, j]), :, int(ah[l, h, j]) - source_head_offset]
                            for j in range(s)], dim=-1)
            yk = fk @ spec["k_weight"][l, h].double().abs() + spec["k_bias"][l, h].double().abs()
            yv = fv @ spec["v_weight"][l, h].double().abs() + spec["v_bias"][l, h].double().abs()
            y1, y2 = yk[:, :half], yk[:, half:]
            c, sn = ct[:, 0], st[:, 0]
            out[0, l, :, h] = torch.cat((y1 * c + y2 * sn, y2 * c + y1 * sn), dim=-1)
            out[1, l, :, h] = yv
    return out


def check_mapped(out: torch.Tensor, ref: torch.Tensor, bound: torch.Tensor, *,
                 abs_factor: float = 2.0 ** -14, rel_norm: float = 1e-2,
                 min_within_ulp: float = 0.999) -> dict:
    """Compare GPU ``out`` with oracle ``ref`` (same dtype); raise AssertionError on failure."""
    assert out.shape == ref.shape and out.dtype == ref.dtype, (out.shape, ref.shape)
    o, r = out.cpu(), ref.cpu()
    diff = (o.double() - r.double()).abs()
    allowed = diff <= abs_factor * bound
    stats = {"elements": o.numel(), "max_abs": float(diff.max()),
             "rel_norm": float(diff.max() / r.double().abs().max().clamp_min(1e-30))}
    mag = r.double().abs()
    sized = (mag > 0) & (mag >= (abs_factor / rel_norm) * bound)
    rel = diff[sized] / mag[sized]
    stats["max_rel_elem"] = float(rel.max()) if rel.numel() else 0.0
    stats["rel_elem_fraction"] = float(sized.double().mean())
    if o.dtype in (torch.bfloat16, torch.float16):
        ulp = ulp_distance(o, r)
        within = ulp <= 1
        stats["within_1ulp"] = float(within.double().mean())
        stats["max_ulp"] = int(ulp.max())
        ok = within | allowed
    else:
        stats["within_1ulp"] = float(allowed.double().mean())
        ok = allowed
    bad = int((~ok).sum())
    stats["violations"] = bad
    assert bad == 0, f"{bad} elements outside tolerance: {stats}"
    assert stats["rel_norm"] <= rel_norm, stats
    assert stats["max_rel_elem"] <= rel_norm, stats
    assert stats["within_1ulp"] >= min_within_ulp, stats
    return stats
