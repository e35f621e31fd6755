"""GPU parity of the fused HIP handoff path against the oracle and golden vectors.

Tolerance (bf16 outputs): each element within 1 bf16 ulp of the oracle, or
within 2^-14 of its summand-magnitude bound (near-cancelling outputs, see
``oracle/tolerance.py``); at least 99.9% within 1 ulp; normwise relative
error <= 1e-2. fp32 outputs: within 2^-18 of the magnitude bound. Slot
addressing and untouched rows: bit-exact.
"""

from __future__ import annotations

import json

import pytest
import torch
from safetensors.torch import load_file

from cachebridge_amd import synthetic
from cachebridge_amd.mapper import HeadwiseMapper, PageMapper
from cachebridge_amd.online.blocks import map_install_block, map_write_block, pack_source_block
from oracle import install as oi
from oracle import tolerance as ot

pytestmark = pytest.mark.gpu

SPEC_KEYS = ("assign_layer", "assign_head", "k_weight", "v_weight", "k_bias", "v_bias")


def _golden(golden_dir, name):
    man = json.loads((golden_dir / "manifest.json").read_text())["files"][name + ".safetensors"]
    return man, load_file(str(golden_dir / f"{name}.safetensors"))


def _factor(dtype):
    return 2.0 ** -14 if dtype == torch.bfloat16 else 2.0 ** -18


@pytest.mark.parametrize("name", ["toy_fp32", "slice_bf16_s1", "slice_bf16_yarn"])
def test_map_page_matches_reference_golden(golden_dir, name):
    man, g = _golden(golden_dir, name)
    spec = {k: g[k] for k in SPEC_KEYS}
    yarn = man.get("yarn")
    mapper = HeadwiseMapper.from_assignment(
        **spec, source_rope_theta=man["source_theta"], target_rope_theta=man["target_theta"],
        source_rope_scaling=yarn, target_rope_scaling=yarn, dtype=g["page"].dtype,
        device="cuda", max_positions=41000)
    page = g["page"].cuda()
    before = page.clone()
    out = mapper.map_page(page, position_start=man["position_start"], output_device="cuda")
    assert torch.equal(page, before)
    bound = ot.magnitude_bound(g["page"], spec, position_start=man["position_start"],
                               source_theta=man["source_theta"], target_thetas=man["target_theta"],
                               source_scaling=yarn, target_scaling=yarn)
    stats = ot.check_mapped(out, g["out"], bound, abs_factor=_factor(g["page"].dtype))
    print(name, stats)


def test_toy_golden_installed_through_a_random_block_table(golden_dir):
    """The toy configuration (8x2 -> 12x2, D 64, 256 fp32 tokens) through the
    paged install: the reference's golden source page is mapped straight into
    a page-16 target pool through a seeded random-permutation block table over
    three times the pages the request needs. The rows at the block table's
    slots must equal the reference's golden ``map_page`` output to the fp32
    parity bar, and every other row of the pool must keep its bits."""
    from cachebridge_amd.plan import rows_from_page
    from cachebridge_amd.pool import PagedKVPool, pool_rows

    man, g = _golden(golden_dir, "toy_fp32")
    spec = {k: g[k] for k in SPEC_KEYS}
    page = g["page"]
    lt, ht = spec["assign_layer"].shape[:2]
    n, dim = page.shape[2], page.shape[4]
    need = (n + 15) // 16
    pages = 3 * need
    mapper = HeadwiseMapper.from_assignment(
        **spec, source_rope_theta=man["source_theta"], target_rope_theta=man["target_theta"],
        dtype=torch.float32, device="cuda", max_positions=4096)
    pool = PagedKVPool(layer_num=lt, pages=pages, head_num=ht, head_dim=dim, page_size=16,
                       dtype=torch.float32, device="cuda", fill=None)
    gen = torch.Generator().manual_seed(77)
    pool.k_data.copy_(torch.randn(pool.k_data.shape, generator=gen))
    pool.v_data.copy_(torch.randn(pool.v_data.shape, generator=gen))
    before_k, before_v = pool.k_data.clone(), pool.v_data.clone()
    bt = torch.randperm(pages, generator=gen)[:need].to(torch.int32)
    slots = synthetic.slots_from_pages(bt, n, 16).cuda()
    source = rows_from_page(page.cuda())
    target = pool_rows(pool, block_table=bt.cuda(), page_size=16, tokens=n)
    mapper.map_install(source, target, num_tokens=n, position_start=man["position_start"])
    torch.cuda.synchronize()
    assert mapper.plan.read_errors() == 0
    got = torch.stack([torch.stack([b[slots] for b in pool.k_buffer]),
                       torch.stack([b[slots] for b in pool.v_buffer])]).cpu()
    bound = ot.magnitude_bound(page, spec, position_start=man["position_start"],
                               source_theta=man["source_theta"], target_thetas=man["target_theta"])
    stats = ot.check_mapped(got, g["out"], bound, abs_factor=_factor(torch.float32))
    print("toy via block table", stats)
    rest = torch.ones(pool.k_buffer[0].shape[0], dtype=torch.bool, device="cuda")
    rest[slots] = False
    for l in range(lt):
        assert torch.equal(pool.k_buffer[l][rest], before_k[l][rest])
        assert torch.equal(pool.v_buffer[l][rest], before_v[l][rest])


def test_reference_artifact_s8_tp_slice_matches_golden(golden_dir):
    man, g = _golden(golden_dir, "slice_bf16_s8")
    files = [{"selected": g["selected"], "k_weight": g["k_weight"], "k_bias": g["k_bias"],
              "v_weight": g["v_weight"], "v_bias": g["v_bias"],
              "headwise": torch.tensor(1, dtype=torch.int8)}]
    mapper = PageMapper.from_tensors(files, source_rope_theta=1e4, target_rope_theta=1e6,
                                     target_tp_rank=1, target_tp_size=2, device="cuda",
                                     max_positions=2048)
    output = torch.empty(2, 1, 32, 1, 128, dtype=torch.bfloat16, device="cuda")
    result = mapper.map_page(g["page"].cuda(), position_start=1000, output_device="cuda",
                             output=output)
    assert result.data_ptr() == output.data_ptr()
    compact = mapper.map_page(g["page"][:, :, :, 1:2].cuda(), position_start=1000,
                              source_head_offset=1, output_device="cuda")
    assert torch.equal(compact, result)
    s = len(man["support"])
    spec = {"assign_layer": g["selected"].view(1, 1, s), "assign_head": torch.ones(1, 1, s, dtype=torch.int64),
            "k_weight": g["k_weight"][1:2][None], "v_weight": g["v_weight"][1:2][None],
            "k_bias": g["k_bias"][1:2][None], "v_bias": g["v_bias"][1:2][None]}
    bound = ot.magnitude_bound(g["page"], spec, position_start=1000, source_theta=1e4,
                               target_thetas=1e6)
    print(ot.check_mapped(result, g["out"], bound))


def _cpu_pool(pool):
    p = oi.RowStorePool(pool.layer_num, pool.size, pool.head_num, pool.head_dim, dtype=pool.dtype)
    for l in range(pool.layer_num):
        p.k_buffer[l].copy_(pool.k_buffer[l].cpu())
        p.v_buffer[l].copy_(pool.v_buffer[l].cpu())
    return p


def _oracle_install(h, before):
    sh = h.shape
    tgt_slots = synthetic.slots_from_pages(h.block_table.cpu(), sh.tokens, sh.page_size)
    mapped = oi.map_install_oracle(_cpu_pool(h.source_pool), h.source_slots.cpu().long(), before,
                                   tgt_slots, h.spec, position_start=0,
                                   source_theta=sh.source_theta, target_thetas=sh.target_theta,
                                   windows=sh.windows, prefix_length=sh.tokens)
    return mapped, tgt_slots


def _check_pools(h, expected, mapped, tgt_slots):
    sh = h.shape
    written = torch.zeros(h.target_pool.size, dtype=torch.bool)
    written[tgt_slots] = True
    for kind, bufs, ebufs in ((0, h.target_pool.k_buffer, expected.k_buffer),
                              (1, h.target_pool.v_buffer, expected.v_buffer)):
        for l in range(sh.target_layers):
            got, want = bufs[l].cpu(), ebufs[l]
            # rows outside the request (and outside each layer's window) are untouched
            assert torch.equal(got[~written], want[~written]), (kind, l)
    bound_spec = {k: h.spec[k] for k in SPEC_KEYS}
    src = h.extras["source_values"]
    bound = ot.magnitude_bound(src, bound_spec, position_start=0, source_theta=sh.source_theta,
                               target_thetas=sh.target_theta)
    got = torch.stack([torch.stack([b.cpu()[tgt_slots] for b in h.target_pool.k_buffer]),
                       torch.stack([b.cpu()[tgt_slots] for b in h.target_pool.v_buffer])])
    first = [0 if (sh.windows is None or w is None) else max(0, sh.tokens - (w - 1))
             for w in (sh.windows or [None] * sh.target_layers)]
    # Every kept row of every layer in one comparison: the within-1-ulp share
    # is a statement about the whole install (a one-token window holds too
    # few elements for it on its own); the per-element bound applies to all.
    ot.check_mapped(torch.cat([got[:, l, first[l]:].flatten() for l in range(sh.target_layers)]),
                    torch.cat([mapped[:, l, first[l]:].flatten() for l in range(sh.target_layers)]),
                    torch.cat([bound[:, l, first[l]:].flatten() for l in range(sh.target_layers)]))
    for l in range(sh.target_layers):
        f = first[l]
        if f:
            want_untouched = torch.stack([expected.k_buffer[l][tgt_slots[:f]],
                                          expected.v_buffer[l][tgt_slots[:f]]])
            assert torch.equal(got[:, l, :f], want_untouched)


@pytest.mark.parametrize("name,tokens,layers,tpw", [("tp4", 512, None, 0), ("full", 256, None, 0),
                                                   ("gemma", 1200, None, 0), ("tp4", 2048, 6, 2048)])
def test_fused_pool_install_matches_oracle(name, tokens, layers, tpw):
    """tpw: cap on tokens per workgroup, forcing many workgroups with long segments."""
    print(f"fused install {name} tokens={tokens} layers={layers} tpw={tpw}", flush=True)
    sh = synthetic.shape(name, tokens=tokens)
    if layers is not None:
        sh.target_layers = layers
    if name == "gemma":
        sh.target_layers = 12  # keeps global layers 5 and 11 and their local neighbours
        sh.windows = sh.windows[:12]
        sh.target_theta = sh.target_theta[:12]
        sh.windows = [None if w is None else 1024 for w in sh.windows]
    h = synthetic.make_handoff(sh, target_pages=128, fill_target=None)
    torch.manual_seed(0)
    h.target_pool.k_data.copy_(torch.randn_like(h.target_pool.k_data, dtype=torch.float32))
    h.target_pool.v_data.copy_(torch.randn_like(h.target_pool.v_data, dtype=torch.float32))
    before = _cpu_pool(h.target_pool)
    h.run(tokens_per_workgroup=tpw)
    assert h.mapper.plan.read_errors() == 0
    mapped, tgt_slots = _oracle_install(h, before)
    _check_pools(h, before, mapped, tgt_slots)


def test_blockwise_install_equals_single_launch():
    sh = synthetic.shape("tp4", tokens=640)
    sh.target_layers = 8
    a = synthetic.make_handoff(sh, target_pages=80, fill_target="zeros")
    a.run()
    b = synthetic.make_handoff(sh, target_pages=80, fill_target="zeros")
    for start in range(0, 640, 256):
        b.run(start=start, stop=min(640, start + 256))
    torch.cuda.synchronize()
    assert torch.equal(a.target_pool.k_data, b.target_pool.k_data)
    assert torch.equal(a.target_pool.v_data, b.target_pool.v_data)


def test_pack_then_write_block_equals_fused_install():
    sh = synthetic.shape("tp4", tokens=300)
    sh.target_layers = 6
    h = synthetic.make_handoff(sh, target_pages=64, fill_target="zeros")
    pool = h.source_pool
    idx64 = h.source_slots.long()
    ws = torch.empty(2 * pool.layer_num * 512 * 2 * 128, dtype=torch.bfloat16, device="cuda")
    block = pack_source_block(pool, idx64, start=0, stop=300, workspace=ws, block_tokens=512)
    want = torch.stack([torch.stack([pool.k_buffer[l][idx64] for l in range(pool.layer_num)]),
                        torch.stack([pool.v_buffer[l][idx64] for l in range(pool.layer_num)])])
    assert torch.equal(block, want)
    tgt_slots = synthetic.slots_from_pages(h.block_table.cpu(), 300, 16).cuda()
    other = synthetic.make_handoff(sh, target_pages=64, fill_target="zeros")
    map_write_block(h.mapper, block, other.target_pool, tgt_slots, start=0, source_head_offset=0)
    h.run()
    torch.cuda.synchronize()
    assert torch.equal(other.target_pool.k_data, h.target_pool.k_data)
    assert torch.equal(other.target_pool.v_data, h.target_pool.v_data)


def test_out_of_range_slots_are_flagged_not_written():
    sh = synthetic.shape("tp4", tokens=128)
    sh.target_layers = 2
    h = synthetic.make_handoff(sh, target_pages=16, fill_target="zeros")
    bad = h.source_slots.clone()
    bad[5] = h.source_pool.size + 7  # beyond the pool
    map_install_block(h.mapper, h.source_pool, bad, h.target_pool, start=0, stop=128,
                      block_table=h.block_table, page_size=16)
    flags = h.mapper.plan.read_errors()
    assert flags & 1


@pytest.mark.parametrize("dim,dtype,support,n", [(64, torch.bfloat16, 3, 200), (64, torch.float32, 2, 200),
                                                 (128, torch.bfloat16, 3, 200), (128, torch.bfloat16, 16, 600)])
def test_support_maps_match_oracle(dim, dtype, support, n):
    """Support-s maps at every kernel that takes them: the general kernel (D 64
    bf16 and fp32 I/O) and the support kernel (D 128 bf16: s = 3 over one
    partial 256-token item, and the largest support, s = 16, over two full
    items and a partial one)."""
    print(f"support maps D={dim} {dtype} s={support} n={n}", flush=True)
    g = torch.Generator().manual_seed(11 + dim + support)
    ls, hs, lt, ht, p0 = max(6, support), 2, 3, 2, 300
    layers = torch.stack([torch.randperm(ls, generator=g)[:support] for _ in range(lt * ht)])
    spec = {"assign_layer": layers.view(lt, ht, support),
            "assign_head": torch.randint(0, hs, (lt, ht, support), generator=g),
            "k_weight": torch.randn(lt, ht, support * dim, dim, generator=g) / (support * dim) ** 0.5,
            "v_weight": torch.randn(lt, ht, support * dim, dim, generator=g) / (support * dim) ** 0.5,
            "k_bias": torch.randn(lt, ht, dim, generator=g) * 0.1,
            "v_bias": torch.randn(lt, ht, dim, generator=g) * 0.1}
    mapper = HeadwiseMapper.from_assignment(**spec, source_rope_theta=1e4, target_rope_theta=1e6, dtype=dtype,
                                            device="cuda", max_positions=2048)
    page = torch.randn(2, ls, n, hs, dim, generator=g).to(dtype)
    out = mapper.map_page(page.cuda(), position_start=p0, output_device="cuda")
    virtual = oi.virtual_source_page(page, spec["assign_layer"], spec["assign_head"])
    ref = oi.assignment_mapper(spec, source_rope_theta=1e4, target_rope_theta=1e6).map_page(
        virtual, position_start=p0)
    bound = ot.magnitude_bound(page, spec, position_start=p0, source_theta=1e4, target_thetas=1e6)
    print(ot.check_mapped(out, ref, bound, abs_factor=_factor(dtype)), flush=True)


@pytest.mark.parametrize("support", [1, 2])
def test_pools_beyond_int32_rows_are_rejected_before_launch(support):
    """The streaming (s = 1) and support (s > 1) kernels keep row indices in 32
    bits, so a pool described with more than 2^31 rows is refused on the host
    and nothing is written. (The descriptions cover real, small buffers and the
    identity index only reaches their first rows, so the call would stay in
    bounds even without the check.)"""
    from cachebridge_amd import plan as cplan
    print(f"int32 row guard s={support}", flush=True)
    g = torch.Generator().manual_seed(5 + support)
    ls, hs, lt, ht, n, d = 4, 2, 2, 2, 64, 128
    spec = {"assign_layer": torch.stack([torch.randperm(ls, generator=g)[:support] for _ in range(lt * ht)]).view(lt, ht, support),
            "assign_head": torch.randint(0, hs, (lt, ht, support), generator=g),
            "k_weight": torch.randn(lt, ht, support * d, d, generator=g) / (support * d) ** 0.5,
            "v_weight": torch.randn(lt, ht, support * d, d, generator=g) / (support * d) ** 0.5,
            "k_bias": torch.zeros(lt, ht, d), "v_bias": torch.zeros(lt, ht, d)}
    mapper = HeadwiseMapper.from_assignment(**spec, source_rope_theta=1e4, target_rope_theta=1e4,
                                            dtype=torch.bfloat16, device="cuda", max_positions=256)
    page = torch.randn(2, ls, n, hs, d, generator=g).to(torch.bfloat16).cuda()
    out = torch.zeros(2, lt, n, ht, d, dtype=torch.bfloat16, device="cuda")
    for side in ("source", "target"):
        src, tgt = cplan.rows_from_page(page), cplan.rows_from_page(out)
        (src if side == "source" else tgt).c.rows = 2 ** 31 + 1
        with pytest.raises(ValueError, match="2\\^31"):
            mapper.plan.launch(src, tgt, num_tokens=n, position_start=0)
    torch.cuda.synchronize()
    assert not out.any()
    mapper.plan.launch(cplan.rows_from_page(page), cplan.rows_from_page(out), num_tokens=n, position_start=0)
    torch.cuda.synchronize()
    assert out.any()


def test_support_items_ignore_tokens_per_workgroup():
    """The support kernel's items are fixed 256-token blocks: a launch with a
    larger tokens_per_workgroup writes every token, bit-identically."""
    print("support s8 tokens_per_workgroup", flush=True)
    sh = synthetic.shape("tp4_s8", tokens=600)
    sh.target_layers = 4
    h = synthetic.make_handoff(sh, target_pages=64)
    bufs = h.target_pool.k_buffer + h.target_pool.v_buffer
    for b in bufs:
        b.zero_()
    h.run()
    torch.cuda.synchronize()
    first = [b.clone() for b in bufs]
    for b in bufs:
        b.zero_()
    h.run(tokens_per_workgroup=512)
    torch.cuda.synchronize()
    assert h.mapper.plan.read_errors() == 0
    for a_, b_ in zip(first, bufs):
        assert torch.equal(a_, b_)
    assert all(bool(b.abs().sum() > 0) for b in first)


@pytest.mark.parametrize("dim,dtype,support", [(96, torch.bfloat16, 1), (256, torch.bfloat16, 2),
                                               (80, torch.float16, 1), (128, torch.float32, 1),
                                               (6, torch.bfloat16, 3), (512, torch.float16, 1),
                                               (128, torch.float16, 2)])
def test_generic_head_dims_and_dtypes_match_oracle(dim, dtype, support):
    """Head dims and dtypes outside the MFMA kernels' (bf16 at 64 / 128, fp32
    at 64) run on the generic fp32 kernel: map_page against the oracle."""
    print(f"generic map D={dim} {dtype} s={support}", flush=True)
    g = torch.Generator().manual_seed(17 + dim + support)
    ls, hs, lt, ht, n, p0 = 6, 2, 3, 2, 70, 123
    layers = torch.stack([torch.randperm(ls, generator=g)[:support] for _ in range(lt * ht)])
    spec = {"assign_layer": layers.view(lt, ht, support),
            "assign_head": torch.randint(0, hs, (lt, ht, support), generator=g),
            "k_weight": torch.randn(lt, ht, support * dim, dim, generator=g) / (support * dim) ** 0.5,
            "v_weight": torch.randn(lt, ht, support * dim, dim, generator=g) / (support * dim) ** 0.5,
            "k_bias": torch.randn(lt, ht, dim, generator=g) * 0.1,
            "v_bias": torch.randn(lt, ht, dim, generator=g) * 0.1}
    mapper = HeadwiseMapper.from_assignment(**spec, source_rope_theta=1e4, target_rope_theta=1e6, dtype=dtype,
                                            device="cuda", max_positions=2048)
    assert mapper.plan.info["weight_terms"] == 1  # the generic plan keeps fp32 maps
    page = torch.randn(2, ls, n, hs, dim, generator=g).to(dtype)
    out = mapper.map_page(page.cuda(), position_start=p0, output_device="cuda")
    virtual = oi.virtual_source_page(page, spec["assign_layer"], spec["assign_head"])
    ref = oi.assignment_mapper(spec, source_rope_theta=1e4, target_rope_theta=1e6).map_page(
        virtual, position_start=p0)
    bound = ot.magnitude_bound(page, spec, position_start=p0, source_theta=1e4, target_thetas=1e6)
    print(ot.check_mapped(out, ref, bound, abs_factor=_factor(dtype)), flush=True)


def _generic_shape(tokens):
    return synthetic.Shape("generic96", 8, 2, 6, 2, 96, tokens, torch.bfloat16, [1, 3, 5, 6],
                           target_theta=[1e6, 1e4, 1e4, 1e6, 1e4, 1e4],
                           windows=[None, 64, 64, None, 64, 64], target_pages=64, seed=3)


def test_generic_pool_install_with_windows_matches_oracle():
    """The generic kernel's paged install: windowed layers, two thetas, block
    table; untouched rows bit-exact, mapped rows within the parity bar."""
    print("generic pool install D=96", flush=True)
    sh = _generic_shape(300)
    h = synthetic.make_handoff(sh, target_pages=64, fill_target=None)
    torch.manual_seed(0)
    h.target_pool.k_data.copy_(torch.randn_like(h.target_pool.k_data, dtype=torch.float32))
    h.target_pool.v_data.copy_(torch.randn_like(h.target_pool.v_data, dtype=torch.float32))
    before = _cpu_pool(h.target_pool)
    h.run()
    assert h.mapper.plan.read_errors() == 0
    mapped, tgt_slots = _oracle_install(h, before)
    _check_pools(h, before, mapped, tgt_slots)


def test_generic_batch_equals_per_request_installs():
    print("generic batch D=96", flush=True)
    from cachebridge_amd.pool import pool_rows

    lengths = [40, 100, 17]
    sh = _generic_shape(sum(lengths))
    b = synthetic.make_batch_handoff(sh, lengths, occupancy=0.5)
    pool = b.target_pool
    pool.k_data.zero_()
    pool.v_data.zero_()
    b.run()
    torch.cuda.synchronize()
    batched = (pool.k_data.clone(), pool.v_data.clone())
    pool.k_data.zero_()
    pool.v_data.zero_()
    ps = sh.page_size
    for sp in b.spans:
        e = sp.target_offset // ps
        src = pool_rows(b.source_pool, index=b.source_slots, index_offset=sp.source_offset, tokens=sp.num_tokens)
        tgt = pool_rows(pool, block_table=b.block_table[e:e + (sp.num_tokens + ps - 1) // ps], page_size=ps,
                        tokens=sp.num_tokens)
        b.mapper.map_install(src, tgt, num_tokens=sp.num_tokens, position_start=sp.position_start,
                             prefix_length=sp.prefix_length)
    torch.cuda.synchronize()
    assert b.mapper.plan.read_errors() == 0
    assert torch.equal(pool.k_data, batched[0]) and torch.equal(pool.v_data, batched[1])
    assert bool(batched[0].abs().sum() > 0)


class _LayerPool:
    """An SGLang-style pool: one K and one V tensor per layer (no shared base),
    so launches describe it through a device table of per-layer pointers."""

    def __init__(self, pool):
        self.layer_num, self.start_layer, self.dtype = pool.layer_num, pool.start_layer, pool.dtype
        self.k_buffer = [b.clone() for b in pool.k_buffer]
        self.v_buffer = [b.clone() for b in pool.v_buffer]

    def _get_key_buffer(self, layer):
        return self.k_buffer[layer - self.start_layer]

    def _get_value_buffer(self, layer):
        return self.v_buffer[layer - self.start_layer]


def test_per_layer_pools_on_a_side_stream_match_the_paged_pool():
    """Per-layer pointer tables stay valid while a launch on another stream
    reads them, whatever the current stream allocates meanwhile; the rows
    equal the stride-described pool's bit for bit."""
    print("per-layer pools on a side stream", flush=True)
    sh = synthetic.shape("tp4", tokens=512)
    sh.target_layers = 6
    h = synthetic.make_handoff(sh, target_pages=64, fill_target="zeros")
    src, tgt = _LayerPool(h.source_pool), _LayerPool(h.target_pool)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    torch.cuda._sleep(20_000_000)  # keep the side launch queued behind busy work
    with torch.cuda.stream(side):
        torch.cuda._sleep(20_000_000)
    map_install_block(h.mapper, src, h.source_slots, tgt, start=0, stop=512, block_table=h.block_table,
                      page_size=16, prefix_length=512, stream=side)
    junk = [torch.full((1 << 18,), -1, dtype=torch.int64, device="cuda") for _ in range(16)]
    side.synchronize()
    torch.cuda.synchronize()
    del junk
    h.run()
    torch.cuda.synchronize()
    assert h.mapper.plan.read_errors() == 0
    for l in range(sh.target_layers):
        assert torch.equal(tgt.k_buffer[l], h.target_pool.k_buffer[l])
        assert torch.equal(tgt.v_buffer[l], h.target_pool.v_buffer[l])
    assert bool(tgt.k_buffer[0].abs().sum() > 0)
