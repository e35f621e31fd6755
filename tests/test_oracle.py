"""The oracle pinned against the reference's golden vectors and closed forms (CPU).

Every check here is on the oracle (and the product's host-side RoPE tables):
golden outputs written from the reference must be reproduced bit for bit;
closed forms (identity maps, exact affine maps, cos^2 + sin^2, fp64 brute
force) pin what the golden vectors leave open; and planted mistakes in the
oracle's computation must fail the same comparisons.
"""

from __future__ import annotations

import json
import math

import pytest
import torch
from safetensors.torch import load_file

from cachebridge_amd import rope as product_rope
from oracle import install as oi
from oracle import mapper as om
from oracle import rope as orope
from oracle import tolerance as ot

SPEC_KEYS = ("assign_layer", "assign_head", "k_weight", "v_weight", "k_bias", "v_bias")


def _golden(golden_dir, name):
    man = json.loads((golden_dir / "manifest.json").read_text())["files"]
    return man, load_file(str(golden_dir / name))


# ----------------------------------------------------------------------------- RoPE tables


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("which", ["t10000", "t1000000", "yarn"])
def test_rope_tables_bit_equal_reference_golden(golden_dir, dim, which):
    man, t = _golden(golden_dir, "rope_tables.safetensors")
    pos = t["positions"]
    if which == "yarn":
        kw = dict(theta=1e6, scaling=man["rope_tables.safetensors"]["yarn"])
    else:
        kw = dict(theta=float(which[1:]), scaling=None)
    c, s = orope.qwen_rope(pos, head_dim=dim, **kw)
    assert torch.equal(c, t[f"cos_d{dim}_{which}"])
    assert torch.equal(s, t[f"sin_d{dim}_{which}"])
    # The product's resident tables (host-built, chunked) hold the same bits.
    pc, ps = product_rope.rope_tables(dim, kw["theta"], kw["scaling"], int(pos.max()) + 1)
    assert torch.equal(pc[pos], t[f"cos_d{dim}_{which}"][:, : dim // 2])
    assert torch.equal(ps[pos], t[f"sin_d{dim}_{which}"][:, : dim // 2])


@pytest.mark.parametrize("scaling", [None, {"rope_type": "yarn", "factor": 4.0,
                                            "original_max_position_embeddings": 32768}])
def test_rope_closed_forms(scaling):
    pos = torch.arange(0, 4096, 7)
    c, s = orope.qwen_rope(pos, head_dim=128, theta=1e6, scaling=scaling)
    mag = 1.0 if scaling is None else 0.1 * math.log(scaling["factor"]) + 1.0
    torch.testing.assert_close(c.square() + s.square(), torch.full_like(c, mag * mag),
                               atol=4e-6, rtol=0)
    # Position 0 is the identity rotation; halves are duplicated.
    assert torch.equal(c[0], torch.full_like(c[0], mag)) and not s[0].any()
    assert torch.equal(c[:, :64], c[:, 64:]) and torch.equal(s[:, :64], s[:, 64:])
    if scaling is None:
        # Pair 0 has inverse frequency 1: phase == position.
        ref = torch.cos(pos.double())
        torch.testing.assert_close(c[:, 0].double(), ref, atol=2e-3, rtol=0)


def test_remove_rope_inverts_apply_rope():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(3, 50, 2, 128, generator=g)
    c, s = orope.qwen_rope(torch.arange(4000, 4050), head_dim=128, theta=1e4)
    y = orope.apply_rope(x, c, s)
    torch.testing.assert_close(orope.remove_rope(y, c, s), x, atol=2e-6, rtol=2e-6)
    # rotate_half is a quarter turn: applying it four times is the identity.
    r = x
    for _ in range(4):
        r = orope.rotate_half(r)
    assert torch.equal(r, x)


# ----------------------------------------------------------------------------- golden maps


def _oracle_map(spec, page, m, *, target_theta=None, transform=None):
    spec = dict(spec)
    if transform is not None:
        spec = transform(spec)
    mapper = oi.assignment_mapper(
        spec, source_rope_theta=m["source_theta"],
        target_rope_theta=m["target_theta"] if target_theta is None else target_theta,
        source_rope_scaling=m.get("yarn"), target_rope_scaling=m.get("yarn"))
    virtual = oi.virtual_source_page(page, spec["assign_layer"], spec["assign_head"])
    return mapper.map_page(virtual, position_start=m["position_start"])


@pytest.mark.parametrize("name", ["toy_fp32", "slice_bf16_s1", "slice_bf16_yarn"])
def test_oracle_reproduces_reference_golden_bit_for_bit(golden_dir, name):
    man, g = _golden(golden_dir, name + ".safetensors")
    m = man[name + ".safetensors"]
    out = _oracle_map({k: g[k] for k in SPEC_KEYS}, g["page"], m)
    assert out.dtype == g["out"].dtype
    assert torch.equal(out, g["out"])


def test_oracle_reference_artifact_s8_tp_slice(golden_dir):
    """Reference-format layer file, unsorted s=8 support, TP 2 rank 1."""
    man, g = _golden(golden_dir, "slice_bf16_s8.safetensors")
    m = man["slice_bf16_s8.safetensors"]
    layer = {"selected": g["selected"], "k_weight": g["k_weight"], "k_bias": g["k_bias"],
             "v_weight": g["v_weight"], "v_bias": g["v_bias"],
             "headwise": torch.tensor(1, dtype=torch.int8)}
    kw = dict(method="cachebridge", source_rope_theta=m["source_theta"],
              target_rope_theta=m["target_theta"], target_tp_rank=m["target_tp_rank"],
              target_tp_size=m["target_tp_size"])
    mapper = om.PageMapper.from_tensors([layer], **kw)
    assert (mapper.target_head_start, mapper.target_head_stop) == (1, 2)
    before = g["page"].clone()
    out = mapper.map_page(g["page"], position_start=m["position_start"])
    assert torch.equal(out, g["out"])
    assert torch.equal(g["page"], before)
    # The head-local mapper on the rank's compact page gives the same bits.
    local = om.HeadLocalPageMapper.from_tensors([layer], **kw)
    compact = local.map_page(g["page"][:, :, :, 1:2], position_start=m["position_start"],
                             source_head_offset=1)
    assert torch.equal(compact, out)


def test_oracle_matches_fp64_brute_force(golden_dir):
    """Toy fp32 configuration against an independent fp64 evaluation."""
    man, g = _golden(golden_dir, "toy_fp32.safetensors")
    m = man["toy_fp32.safetensors"]
    spec = {k: g[k] for k in SPEC_KEYS}
    virtual = oi.virtual_source_page(g["page"], g["assign_layer"], g["assign_head"])
    lt, _, s = g["assign_layer"].shape
    layers = [{"selected": torch.tensor([l * s + k for k in range(s)]),
               "k_weight": spec["k_weight"][l], "k_bias": spec["k_bias"][l],
               "v_weight": spec["v_weight"][l], "v_bias": spec["v_bias"][l]} for l in range(lt)]
    exact = om.brute_force_map(virtual, layers, position_start=m["position_start"],
                               source_theta=m["source_theta"], target_theta=m["target_theta"])
    bound = ot.magnitude_bound(g["page"], spec, position_start=m["position_start"],
                               source_theta=m["source_theta"], target_thetas=m["target_theta"])
    err = (g["out"].double() - exact).abs()
    # fp32 chain: ~ (s*D + 4) roundings of relative size 2^-24 on the summands.
    assert bool((err <= 2.0 ** -16 * bound + 1e-30).all()), float((err / bound).max())


def test_virtual_page_identity_for_head_identity_assignment():
    """Re-indexing the page by assignment == the reference's layer selection."""
    g = torch.Generator().manual_seed(21)
    page = torch.randn(2, 6, 16, 2, 8, generator=g)
    selected = [4, 1]
    lt, ht, d = 2, 2, 8
    al = torch.tensor(selected).expand(lt, ht, 2).contiguous()
    ah = torch.arange(ht)[None, :, None].expand(lt, ht, 2).contiguous()
    w = torch.randn(lt, ht, 2 * d, d, generator=g) / 4
    b = torch.randn(lt, ht, d, generator=g) / 10
    spec = {"assign_layer": al, "assign_head": ah, "k_weight": w, "v_weight": w.flip(-1),
            "k_bias": b, "v_bias": b.flip(-1)}
    via_virtual = oi.assignment_mapper(spec, source_rope_theta=1e4, target_rope_theta=1e6).map_page(
        oi.virtual_source_page(page, al, ah), position_start=9)
    layers = [{"selected": torch.tensor(selected), "k_weight": w[l], "k_bias": b[l],
               "v_weight": w[l].flip(-1), "v_bias": b[l].flip(-1),
               "headwise": torch.tensor(1, dtype=torch.int8)} for l in range(lt)]
    direct = om.PageMapper.from_tensors(layers, method="cachebridge", source_rope_theta=1e4,
                                        target_rope_theta=1e6).map_page(page, position_start=9)
    assert torch.equal(via_virtual, direct)


# ----------------------------------------------------------------------------- planted mistakes


def _transpose_w(spec):
    spec["k_weight"] = spec["k_weight"].transpose(-1, -2).contiguous()
    return spec


def _drop_bias(spec):
    spec["k_bias"] = torch.zeros_like(spec["k_bias"])
    return spec


def _swap_heads(spec):
    spec["assign_head"] = 1 - spec["assign_head"]
    return spec


@pytest.mark.parametrize("mistake", ["transposed_weight", "dropped_bias", "wrong_head",
                                     "wrong_target_theta"])
def test_golden_comparison_rejects_planted_oracle_mistakes(golden_dir, mistake):
    """A plausible slip in the oracle fails the golden check at the parity tolerance."""
    man, g = _golden(golden_dir, "slice_bf16_s1.safetensors")
    m = man["slice_bf16_s1.safetensors"]
    spec = {k: g[k].clone() for k in SPEC_KEYS}
    transform = {"transposed_weight": _transpose_w, "dropped_bias": _drop_bias,
                 "wrong_head": _swap_heads, "wrong_target_theta": None}[mistake]
    theta = 1e4 if mistake == "wrong_target_theta" else None
    bad = _oracle_map(spec, g["page"], m, target_theta=theta, transform=transform)
    bound = ot.magnitude_bound(g["page"], spec, position_start=m["position_start"],
                               source_theta=m["source_theta"], target_thetas=m["target_theta"])
    with pytest.raises(AssertionError):
        ot.check_mapped(bad, g["out"], bound)


def test_tolerance_accepts_one_ulp_and_rejects_two():
    g = torch.Generator().manual_seed(5)
    ref = (torch.randn(2, 1, 64, 2, 128, generator=g) * 3).to(torch.bfloat16)
    bits = ref.view(torch.int16)
    one = (bits + 1).view(torch.bfloat16)
    assert int(ot.bf16_ulp_distance(one, ref).max()) == 1
    tiny = torch.zeros(ref.shape, dtype=torch.float64)
    ot.check_mapped(one, ref, tiny, min_within_ulp=1.0)
    two = (bits + 2).view(torch.bfloat16)
    with pytest.raises(AssertionError):
        ot.check_mapped(two, ref, tiny)


@pytest.mark.parametrize("dtype,mant", [(torch.bfloat16, 7), (torch.float16, 10)])
def test_ulp_distance_counts_representable_steps(dtype, mant):
    """One step up from a normal x is 2^(floor(log2|x|) - mantissa bits); the
    distance counts steps across zero (+0 and -0 coincide)."""
    x = torch.tensor([1.0, 2.5, 3e-3, 700.0, 0.75], dtype=dtype)
    up = (x.view(torch.int16) + 1).view(dtype)
    step = up.double() - x.double()
    expect = torch.exp2(torch.floor(torch.log2(x.double())) - mant)
    assert torch.equal(step, expect)
    assert ot.ulp_distance(up, x).tolist() == [1] * 5
    three = (x.view(torch.int16) + 3).view(dtype)
    assert ot.ulp_distance(three, x).tolist() == [3] * 5
    zeros = torch.tensor([0.0, -0.0], dtype=dtype)
    assert ot.ulp_distance(zeros[:1], zeros[1:]).item() == 0
    tiny = torch.tensor([1], dtype=torch.int16).view(dtype)   # smallest positive
    neg = torch.tensor([-32767], dtype=torch.int16).view(dtype)  # bits 0x8001: smallest negative
    assert ot.ulp_distance(tiny, neg).item() == 2


def test_tolerance_accepts_one_fp16_ulp_and_rejects_two():
    g = torch.Generator().manual_seed(6)
    ref = (torch.randn(2, 1, 32, 2, 96, generator=g) * 3).to(torch.float16)
    bits = ref.view(torch.int16)
    tiny = torch.zeros(ref.shape, dtype=torch.float64)
    ot.check_mapped((bits + 1).view(torch.float16), ref, tiny, min_within_ulp=1.0)
    with pytest.raises(AssertionError):
        ot.check_mapped((bits + 2).view(torch.float16), ref, tiny)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_row_store_writes_exactly_its_inputs_at_loc(dtype):
    """The oracle's SGLang row-store stand-in (``set_kv_buffer``): the rows at
    ``loc`` of the named layer become exactly the given K and V rows (cast to
    the pool dtype when they arrive in another), every other row of that layer
    and every row of every other layer keep their bits, for int64 and int32
    ``loc`` in any order. The first property is the one the reference asserts
    after its own installs through SGLang's pool
    (``rt/clean_adapter.py:638-652``: ``_get_key_buffer(layer)[indices]`` and
    ``_get_value_buffer(layer)[indices]`` bit-equal the written values, layer
    by layer, ``rt/`` = ``src/cachebridge/backends/sglang/runtime/``)."""
    g = torch.Generator().manual_seed(31)
    layers, rows, heads, dim = 3, 40, 2, 8
    fill = torch.randn(2, layers, rows, heads, dim, generator=g).to(dtype)
    pool = oi.RowStorePool(layers, rows, heads, dim, dtype=dtype, start_layer=2, fill=fill)
    before_k = [b.clone() for b in pool.k_buffer]
    before_v = [b.clone() for b in pool.v_buffer]
    loc = torch.randperm(rows, generator=g)[:11]
    k = torch.randn(11, heads, dim, generator=g, dtype=torch.float32)
    v = torch.randn(11, heads, dim, generator=g, dtype=torch.float32)
    for index in (loc, loc.to(torch.int32)):
        pool.set_kv_buffer(None, index, k, v, layer_id_override=3)
        assert torch.equal(pool._get_key_buffer(3)[loc.long()], k.to(dtype))
        assert torch.equal(pool._get_value_buffer(3)[loc.long()], v.to(dtype))
        rest = torch.ones(rows, dtype=torch.bool)
        rest[loc.long()] = False
        for i in range(layers):
            kb, vb = pool.k_buffer[i], pool.v_buffer[i]
            if i == 1:  # layer 3 (start_layer 2): only the rows at loc changed
                assert torch.equal(kb[rest], before_k[i][rest]) and torch.equal(vb[rest], before_v[i][rest])
            else:
                assert torch.equal(kb, before_k[i]) and torch.equal(vb, before_v[i])
    # A duplicate-free loc in the pool dtype is stored bit for bit.
    k2 = torch.randn(11, heads, dim, generator=g).to(dtype)
    pool.set_kv_buffer(None, loc, k2, k2, layer_id_override=2)
    assert torch.equal(pool._get_key_buffer(2)[loc], k2)
    assert torch.equal(pool._get_value_buffer(2)[loc], k2)
