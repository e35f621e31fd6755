"""Seeded synthetic handoff workloads at the benchmark shapes.

Every tensor is generated on the CPU with a seeded ``torch.Generator`` (so a
workload is reproducible across machines) and then placed on the device.

Shapes (source model -> target model, per GPU):

- ``toy``:     source 8x2 -> target 12x2, head_dim 64, 256 tokens, fp32.
- ``tp4``:     Qwen3-14B -> 32B, one TP4 rank: source 40x2 -> target 64x2,
               head_dim 128, 4096 tokens, bf16, 65536-page pool.
- ``full``:    Qwen3-14B -> 32B whole model: 40x8 -> 64x8, 4096 tokens.
- ``full32k``: 40x8 -> 64x8, 32768 tokens, each source head feeding ~4 targets.
- ``gemma``:   source 40x8 -> Gemma-3-style target 62x16, 5:1 local/global,
               sliding window 1024 on local layers, head map h_src = h // 2,
               8192 tokens, theta 1e4 local / 1e6 global.
- ``batch``:   64 ragged requests (lognormal lengths, median 2048, sigma 0.5,
               clipped to [256, 16384]; 137,440 tokens) at the TP4 share
               (40x2 -> 64x2) into one shared target pool at 85% occupancy
               (0.99 M slots; the 64x8 pool at that occupancy would need
               260 GB next to the source pool, more than one GPU holds).
- ``batch_full``: the same requests at the whole-model 64x8 geometry, with the
               target pool at 50% occupancy (2x the batch's pages).
- ``tp4_s8`` / ``full_s8``: the shipped support-8 recipe's structure at the
               TP4 share and the whole model: every target layer reads 8
               distinct source layers (its depth-matched layer first, then 7
               seeded neighbours within 12 layers), shared by K and V and by
               every head, with head identity; maps are [8*128, 128].

Source keys are treated as stored RoPE-rotated (as SGLang stores them); the
map is A ~ N(0, 1/(s*D)), b ~ N(0, 0.01); bf16 sources are N(0,1) times a
per-channel lognormal(0, 0.5) scale.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from .layouts import head_assignment
from .mapper import HeadwiseMapper
from .pool import PagedKVPool


@dataclass
class Shape:
    name: str
    source_layers: int
    source_heads: int
    target_layers: int
    target_heads: int
    head_dim: int
    tokens: int
    dtype: torch.dtype
    selected: list
    source_theta: float = 1e6
    target_theta: object = 1e6           # float or per-target-layer list
    windows: list | None = None          # per-target-layer None / sliding window size
    head_map: str = "random"             # "random" or "half" (h_src = h // 2)
    target_pages: int | None = None
    page_size: int = 16
    seed: int = 0
    support: int = 1                     # source (layer, head) pairs per target (support-s maps)


def shape(name: str, tokens: int | None = None) -> Shape:
    sel16 = [round(x) for x in torch.linspace(0, 39, 16).tolist()]
    if name == "toy":
        s = Shape("toy", 8, 2, 12, 2, 64, 256, torch.float32, [], 1e4, 1e6, seed=1)
    elif name == "tp4":
        s = Shape("tp4", 40, 2, 64, 2, 128, 4096, torch.bfloat16, sel16, target_pages=65536, seed=2)
    elif name == "full":
        s = Shape("full", 40, 8, 64, 8, 128, 4096, torch.bfloat16, sel16, target_pages=8192, seed=3)
    elif name == "full32k":
        s = Shape("full32k", 40, 8, 64, 8, 128, 32768, torch.bfloat16, sel16, target_pages=4096, seed=4)
    elif name == "gemma":
        lt = 62
        glob = [(i + 1) % 6 == 0 for i in range(lt)]
        s = Shape("gemma", 40, 8, lt, 16, 128, 8192, torch.bfloat16, sel16,
                  target_theta=[1e6 if g else 1e4 for g in glob],
                  windows=[None if g else 1024 for g in glob], head_map="half",
                  target_pages=1024, seed=5)
    elif name in ("tp4_s8", "full_s8"):
        heads = 2 if name == "tp4_s8" else 8
        s = Shape(name, 40, heads, 64, heads, 128, 4096, torch.bfloat16, [], head_map="identity",
                  target_pages=65536 if name == "tp4_s8" else 8192, seed=8 if name == "tp4_s8" else 9,
                  support=8)
    elif name in ("batch", "batch_full"):
        heads = 2 if name == "batch" else 8
        s = Shape(name, 40, heads, 64, heads, 128, sum(request_lengths()), torch.bfloat16, sel16,
                  seed=6 if name == "batch" else 7)
    else:
        raise ValueError(f"unknown workload shape {name!r}")
    if tokens is not None:
        s.tokens = tokens
    return s


def request_lengths(count: int = 64, median: int = 2048, sigma: float = 0.5, lo: int = 256,
                    hi: int = 16384, seed: int = 77) -> list[int]:
    """Seeded ragged request lengths: round(median * exp(sigma * N(0,1))) clipped to [lo, hi]."""
    g = torch.Generator().manual_seed(seed)
    x = torch.exp(torch.randn(count, generator=g, dtype=torch.float64) * sigma) * median
    return x.round().clamp(lo, hi).long().tolist()


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def mapper_spec(sh: Shape) -> dict:
    """Assignment and fp32 maps of a shape (CPU tensors)."""
    g = _gen(1000 + sh.seed)
    lt, ht, d = sh.target_layers, sh.target_heads, sh.head_dim
    if sh.support > 1:
        return _support_spec(sh, g)
    if sh.selected:
        selected = list(sh.selected)
    else:
        selected = sorted(torch.randperm(sh.source_layers, generator=g)[:4].tolist())
    pick = torch.randint(0, len(selected), (lt, ht, 1), generator=g)
    layer = torch.tensor(selected, dtype=torch.int64)[pick]
    if sh.head_map == "half":  # Gemma-style: target head h reads source head h // 2
        heads = head_assignment(sh.source_heads, ht, [h // 2 for h in range(ht)])
        head = torch.tensor(heads, dtype=torch.int64).view(1, ht, 1).expand(lt, ht, 1).clone()
    else:
        head = torch.randint(0, sh.source_heads, (lt, ht, 1), generator=g)
    std = 1.0 / math.sqrt(d)
    return {
        "assign_layer": layer,
        "assign_head": head,
        "k_weight": torch.randn(lt, ht, d, d, generator=g) * std,
        "v_weight": torch.randn(lt, ht, d, d, generator=g) * std,
        "k_bias": torch.randn(lt, ht, d, generator=g) * 0.1,
        "v_bias": torch.randn(lt, ht, d, generator=g) * 0.1,
        "selected": selected,
    }


def support_layers(sh: Shape, g: torch.Generator) -> list[list[int]]:
    """Per target layer, ``sh.support`` distinct source layers: the depth-matched
    layer first, then seeded neighbours within 12 layers (the recipe's shape)."""
    out = []
    ls, lt = sh.source_layers, sh.target_layers
    for l in range(lt):
        c = round(l * (ls - 1) / max(lt - 1, 1))
        near = [x for x in range(max(0, c - 12), min(ls, c + 13)) if x != c]
        pick = torch.randperm(len(near), generator=g)[: sh.support - 1].tolist()
        out.append([c] + [near[i] for i in pick])
    return out


def _support_spec(sh: Shape, g: torch.Generator) -> dict:
    lt, ht, d, s = sh.target_layers, sh.target_heads, sh.head_dim, sh.support
    layers = torch.tensor(support_layers(sh, g), dtype=torch.int64)      # [lt, s]
    std = 1.0 / math.sqrt(s * d)
    return {
        "assign_layer": layers[:, None, :].expand(lt, ht, s).clone(),
        "assign_head": torch.tensor(head_assignment(sh.source_heads, ht, list(range(ht))), dtype=torch.int64)
        .view(1, ht, 1).expand(lt, ht, s).clone(),
        "k_weight": torch.randn(lt, ht, s * d, d, generator=g) * std,
        "v_weight": torch.randn(lt, ht, s * d, d, generator=g) * std,
        "k_bias": torch.randn(lt, ht, d, generator=g) * 0.1,
        "v_bias": torch.randn(lt, ht, d, generator=g) * 0.1,
        "selected": sorted({int(x) for x in layers.flatten()}),
    }


def make_mapper(sh: Shape, spec: dict | None = None, device="cuda", max_positions=None) -> HeadwiseMapper:
    spec = spec if spec is not None else mapper_spec(sh)
    return HeadwiseMapper.from_assignment(
        assign_layer=spec["assign_layer"], assign_head=spec["assign_head"],
        k_weight=spec["k_weight"], k_bias=spec["k_bias"],
        v_weight=spec["v_weight"], v_bias=spec["v_bias"],
        source_rope_theta=sh.source_theta, target_rope_theta=sh.target_theta,
        windows=sh.windows, dtype=sh.dtype, device=device,
        max_positions=max_positions or max(40960, sh.tokens),
    )


def source_values(sh: Shape, tokens: int | None = None) -> torch.Tensor:
    """``[2, Ls, tokens, Hs, D]`` CPU source K/V in the shape's dtype."""
    g = _gen(2000 + sh.seed)
    n = sh.tokens if tokens is None else tokens
    x = torch.randn(2, sh.source_layers, n, sh.source_heads, sh.head_dim, generator=g)
    if sh.dtype == torch.bfloat16:
        scale = torch.exp(torch.randn(sh.head_dim, generator=g) * 0.5)
        x = x * scale
    return x.to(sh.dtype)


def fragmented_pages(total_pages: int, needed: int, seed: int) -> torch.Tensor:
    """First ``needed`` entries of a seeded-shuffled free list of ``total_pages`` pages."""
    if needed > total_pages:
        raise ValueError("pool too small for the request")
    return torch.randperm(total_pages, generator=_gen(seed))[:needed].to(torch.int32)


def slots_from_pages(pages: torch.Tensor, tokens: int, page_size: int) -> torch.Tensor:
    t = torch.arange(tokens, dtype=torch.int64)
    return (pages.long()[t // page_size] * page_size + t % page_size)


@dataclass
class Handoff:
    """One resident handoff: source pool + slots, target pool + block table, mapper."""

    shape: Shape
    spec: dict
    mapper: HeadwiseMapper
    source_pool: PagedKVPool
    source_slots: torch.Tensor         # int32 [tokens] rows of the source pool
    target_pool: PagedKVPool
    block_table: torch.Tensor          # int32 [ceil(tokens / page_size)]
    extras: dict = field(default_factory=dict)

    @property
    def tokens(self) -> int:
        return self.shape.tokens

    def run(self, *, start: int = 0, stop: int | None = None, stream=None, tokens_per_workgroup=0):
        from .online.blocks import map_install_block

        stop = self.tokens if stop is None else stop
        map_install_block(self.mapper, self.source_pool, self.source_slots, self.target_pool,
                          start=start, stop=stop, block_table=self.block_table,
                          page_size=self.shape.page_size, prefix_length=self.tokens,
                          stream=stream, tokens_per_workgroup=tokens_per_workgroup)


def make_handoff(sh: Shape, device="cuda", *, target_pages: int | None = None,
                 fill_target: str | None = None, source: torch.Tensor | None = None,
                 device_source: bool = False) -> Handoff:
    """Build a resident handoff of shape ``sh`` on ``device``.

    Source values come from ``source_values`` (CPU generator), or with
    ``device_source`` are drawn on the device from a seeded generator (same
    distribution; fast for multi-GB pools, ``extras["source_values"]`` is then
    None and the rows are read back from the pool where needed).
    """
    spec = mapper_spec(sh)
    mapper = make_mapper(sh, spec, device=device)
    ps = sh.page_size
    n = sh.tokens
    src_pages_needed = (n + ps - 1) // ps
    src_total = src_pages_needed * 2
    src_pool = PagedKVPool(layer_num=sh.source_layers, pages=src_total, head_num=sh.source_heads,
                           head_dim=sh.head_dim, page_size=ps, dtype=sh.dtype, device=device)
    src_page_list = fragmented_pages(src_total, src_pages_needed, 3000 + sh.seed)
    src_slots = slots_from_pages(src_page_list, n, ps)
    src_slots_d = src_slots.to(device)
    if device_source and source is None:
        values = None
        g = torch.Generator(device=device).manual_seed(5000 + sh.seed)
        scale = torch.ones(sh.head_dim)
        if sh.dtype == torch.bfloat16:
            scale = torch.exp(torch.randn(sh.head_dim, generator=_gen(2000 + sh.seed)) * 0.5)
        scale = scale.to(device)
        for l in range(sh.source_layers):
            for buf in (src_pool.k_buffer[l], src_pool.v_buffer[l]):
                x = torch.randn((n, sh.source_heads, sh.head_dim), generator=g, device=device)
                buf[src_slots_d] = (x * scale).to(sh.dtype)
    else:
        values = source if source is not None else source_values(sh)
        for l in range(sh.source_layers):
            src_pool.k_buffer[l][src_slots_d] = values[0, l].to(device)
            src_pool.v_buffer[l][src_slots_d] = values[1, l].to(device)
    pages = target_pages or sh.target_pages or max(src_pages_needed * 2, 64)
    tgt_pool = PagedKVPool(layer_num=sh.target_layers, pages=pages, head_num=sh.target_heads,
                           head_dim=sh.head_dim, page_size=ps, dtype=sh.dtype, device=device,
                           fill=fill_target)
    bt = fragmented_pages(pages, src_pages_needed, 4000 + sh.seed)
    return Handoff(sh, spec, mapper, src_pool, src_slots_d.to(torch.int32), tgt_pool,
                   bt.to(device), extras={"source_values": values})


def algorithmic_bytes(sh: Shape, tokens_per_layer: list | None = None) -> int:
    """Bytes a handoff must move at minimum: target writes, distinct source reads once,
    fp32-equivalent weights once, and the token index."""
    e = 2 if sh.dtype == torch.bfloat16 else 4
    d = sh.head_dim
    spec = mapper_spec(sh)
    pairs = {(int(l), int(h)) for l, h in zip(spec["assign_layer"].flatten(),
                                               spec["assign_head"].flatten())}
    if tokens_per_layer is None:
        tokens_per_layer = [window_tokens(sh, l) for l in range(sh.target_layers)]
    write = 2 * e * d * sum(t * sh.target_heads for t in tokens_per_layer)
    read = 2 * e * d * len(pairs) * sh.tokens
    weights = 4 * 2 * sh.target_layers * sh.target_heads * (sh.support * d * d + d)
    return write + read + weights + 8 * sh.tokens


def window_tokens(sh: Shape, layer: int) -> int:
    w = None if sh.windows is None else sh.windows[layer]
    return sh.tokens if w is None else min(sh.tokens, w - 1)


def algorithmic_flops(sh: Shape) -> int:
    d = sh.head_dim
    return sum(2 * 2 * window_tokens(sh, l) * sh.target_heads * sh.support * d * d
               for l in range(sh.target_layers))


@dataclass
class BatchHandoff:
    """A resident ragged batch: one source pool, one shared target pool, one span per request."""

    shape: Shape
    spec: dict
    mapper: HeadwiseMapper
    source_pool: PagedKVPool
    source_slots: torch.Tensor     # int32, the requests' source slots back to back
    target_pool: PagedKVPool
    block_table: torch.Tensor      # int32, the requests' pages back to back
    spans: list                    # plan.RequestSpan per request
    lengths: list

    @property
    def tokens(self) -> int:
        return sum(self.lengths)

    def run(self, *, stream=None, tokens_per_workgroup=0):
        from .online.blocks import map_install_batch

        if tokens_per_workgroup:
            raise ValueError("batched launches use one workgroup per CU")
        map_install_batch(self.mapper, self.source_pool, self.source_slots, self.target_pool,
                          self.spans, block_table=self.block_table,
                          page_size=self.shape.page_size, stream=stream)


def make_batch_handoff(sh: Shape, lengths: list | None = None, *, occupancy: float | None = None,
                       device="cuda") -> BatchHandoff:
    """Requests of ``lengths`` tokens (whole histories at positions 0..n-1) in shared pools.

    The target pool is sized so that the batch's pages are the free
    ``1 - occupancy`` of it, drawn from a seeded shuffled free list. Source
    values are drawn on the device from a seeded generator (bf16 N(0,1) times
    the per-channel lognormal scale), which keeps multi-GB pools fast to build.
    """
    from .plan import RequestSpan

    lengths = list(lengths if lengths is not None else request_lengths())
    if occupancy is None:
        occupancy = 0.85 if sh.name == "batch" else 0.5
    ps = sh.page_size
    total = sum(lengths)
    spec = mapper_spec(sh)
    mapper = make_mapper(sh, spec, device=device, max_positions=max(40960, max(lengths)))
    need = sum((n + ps - 1) // ps for n in lengths)
    src_total = need * 2
    src_pool = PagedKVPool(layer_num=sh.source_layers, pages=src_total, head_num=sh.source_heads,
                           head_dim=sh.head_dim, page_size=ps, dtype=sh.dtype, device=device)
    g = torch.Generator(device=device).manual_seed(5000 + sh.seed)
    scale = torch.exp(torch.randn(sh.head_dim, generator=_gen(2000 + sh.seed)) * 0.5).to(device)
    src_pages = fragmented_pages(src_total, need, 3000 + sh.seed)
    slots, spans, entry, off = [], [], 0, 0
    for n in lengths:
        k = (n + ps - 1) // ps
        slots.append(slots_from_pages(src_pages[entry:entry + k], n, ps))
        spans.append(RequestSpan(off, entry * ps, n, 0, 0))
        entry += k
        off += n
    src_slots = torch.cat(slots).to(device)
    for l in range(sh.source_layers):
        for buf in (src_pool.k_buffer[l], src_pool.v_buffer[l]):
            x = torch.randn((total, sh.source_heads, sh.head_dim), generator=g, device=device)
            buf[src_slots] = (x * scale).to(sh.dtype)
    pages = max(int(math.ceil(need / (1.0 - occupancy))), need)
    tgt_pool = PagedKVPool(layer_num=sh.target_layers, pages=pages, head_num=sh.target_heads,
                           head_dim=sh.head_dim, page_size=ps, dtype=sh.dtype, device=device)
    bt = fragmented_pages(pages, need, 4000 + sh.seed).to(device)
    return BatchHandoff(sh, spec, mapper, src_pool, src_slots.to(torch.int32), tgt_pool, bt,
                        spans, lengths)
