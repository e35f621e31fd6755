"""Seeded random model pairs through the fused install, against the oracle.

Each case draws a source and target geometry (layers, heads, selected source
layers, a random head assignment), head_dim and dtype, a token count that is
not a multiple of the 16- and 32-token sub-tiles, the page size, per-layer
target thetas, sliding windows on some layers and a cap on tokens per
workgroup. The unit structure (one- and two-job units, groups read by a
single unit, several window classes, segments crossing units) then differs
from the configured workloads. Rows outside the request and outside each
layer's window stay bit-identical; mapped rows meet the oracle tolerance
(module docstring of ``test_gpu_parity``).
"""

from __future__ import annotations

import random

import pytest
import torch

from cachebridge_amd import synthetic

from .test_gpu_batch import _batch, check_batch_equals_single
from .test_gpu_parity import _check_pools, _cpu_pool, _oracle_install

pytestmark = pytest.mark.gpu

GEOMETRIES = [(128, torch.bfloat16), (128, torch.bfloat16), (64, torch.bfloat16), (64, torch.float32),
              (96, torch.bfloat16)]


def random_shape(seed: int):
    """A seeded random handoff shape and tokens-per-workgroup cap."""
    r = random.Random(seed)
    d, dtype = r.choice(GEOMETRIES)
    ls, hs = r.randint(3, 12), r.randint(1, 4)
    lt, ht = r.randint(2, 9), r.randint(1, 5)
    selected = sorted(r.sample(range(ls), r.randint(1, min(ls, 6))))
    windows = None
    if r.random() < 0.5:  # at most 4 window classes (full history included)
        windows = [None if r.random() < 0.4 else r.choice([2, 129, 300]) for _ in range(lt)]
    # Support-s maps (s source pairs per target, head identity) where the
    # source has the heads and layers for them.
    support = r.choice([1, 1, 1, 2, 3]) if hs >= ht and ls >= 4 else 1
    sh = synthetic.Shape(f"random{seed}", ls, hs, lt, ht, d, r.randint(1, 700), dtype, selected,
                         source_theta=r.choice([1e4, 1e6]),
                         target_theta=[r.choice([1e4, 1e6]) for _ in range(lt)],
                         windows=windows, head_map="identity" if support > 1 else "random",
                         page_size=r.choice([1, 16]), seed=100 + seed, support=support)
    # The general support-s kernel at D 64 takes caps in 128-token steps.
    return sh, r.choice([0, 256] if support > 1 else [0, 0, 64, 256])


@pytest.mark.parametrize("seed", range(48))
def test_random_shapes_match_oracle(seed):
    sh, tpw = random_shape(seed)
    print(f"random shape {seed}: s={sh.support} {sh.source_layers}x{sh.source_heads} -> {sh.target_layers}x"
          f"{sh.target_heads} D={sh.head_dim} {sh.dtype} T={sh.tokens} page={sh.page_size} "
          f"windows={sh.windows} tpw={tpw}", flush=True)
    h = synthetic.make_handoff(sh, fill_target=None)
    g = torch.Generator(device="cuda").manual_seed(seed)
    for data in (h.target_pool.k_data, h.target_pool.v_data):
        data.copy_(torch.randn(data.shape, generator=g, device="cuda").to(data.dtype))
    before = _cpu_pool(h.target_pool)
    h.run(tokens_per_workgroup=tpw)
    assert h.mapper.plan.read_errors() == 0
    mapped, tgt_slots = _oracle_install(h, before)
    _check_pools(h, before, mapped, tgt_slots)


@pytest.mark.parametrize("seed", range(24))
def test_random_batches_equal_per_request_installs(seed):
    """A random ragged batch (empty requests, offsets into the prefix, prefixes
    beyond the block) over a random model pair, in one launch, against one
    launch per request, bit for bit."""
    sh, _ = random_shape(1000 + seed)
    sh.page_size = 16
    r = random.Random(seed)
    count = r.randint(1, 12)
    lengths = [r.choice([0, r.randint(1, 40), r.randint(1, 400)]) for _ in range(count)]
    positions = [r.choice([0, r.randint(0, 500)]) for _ in range(count)]
    prefixes = [r.choice([0, p + n + r.randint(0, 300)]) for n, p in zip(lengths, positions)]
    sh.tokens = max(1, sum(lengths))
    print(f"random batch {seed}: s={sh.support} {sh.source_layers}x{sh.source_heads} -> "
          f"{sh.target_layers}x{sh.target_heads} D={sh.head_dim} {sh.dtype} windows={sh.windows} "
          f"lengths={lengths} positions={positions} prefixes={prefixes}", flush=True)
    pages = sum((n + 15) // 16 for n in lengths) * 2 + 2
    h = synthetic.make_handoff(sh, target_pages=pages, fill_target="zeros")
    spans, bt = _batch(lengths, positions, prefixes, pages, seed=seed)
    check_batch_equals_single(h, spans, bt.to(h.target_pool.device))


# Large supports through the support kernel (bf16, head_dim 128): window
# classes holding fewer jobs than there are XCDs, an odd number of keys and
# values jobs per class (the plan's per-XCD placement of keys and values
# runs then takes its fallback on some classes), members that are not in
# layer order (the kernel visits them sorted), and a partial last item.
@pytest.mark.parametrize("ls,hs,lt,ht,support,windows,tokens,page", [
    (16, 3, 7, 3, 8, [None, 300, None, 129, 300, None, 2], 700, 16),
    (20, 1, 3, 1, 12, None, 520, 1),
    (12, 2, 5, 2, 8, [300, None, 300, None, 129], 300, 16),
])
def test_large_supports_match_oracle(ls, hs, lt, ht, support, windows, tokens, page):
    print(f"support {support}: {ls}x{hs} -> {lt}x{ht} T={tokens} page={page} windows={windows}", flush=True)
    sh = synthetic.Shape(f"support{support}_{lt}x{ht}", ls, hs, lt, ht, 128, tokens, torch.bfloat16,
                         list(range(ls)), source_theta=1e4, target_theta=[1e6] * lt, windows=windows,
                         head_map="identity", page_size=page, seed=300 + support + lt, support=support)
    h = synthetic.make_handoff(sh, fill_target=None)
    g = torch.Generator(device="cuda").manual_seed(support + lt)
    for data in (h.target_pool.k_data, h.target_pool.v_data):
        data.copy_(torch.randn(data.shape, generator=g, device="cuda").to(data.dtype))
    before = _cpu_pool(h.target_pool)
    h.run()
    assert h.mapper.plan.read_errors() == 0
    mapped, tgt_slots = _oracle_install(h, before)
    _check_pools(h, before, mapped, tgt_slots)
