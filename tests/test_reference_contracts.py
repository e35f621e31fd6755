"""The reference's own tests for this path, restated (CPU).

Mapper contracts run on the oracle (the product mapper needs a GPU; the GPU
parity tests hold it to the oracle). Host logic that the product implements
itself (leases, the unpublished transaction, run geometry, head ownership,
windows) is tested directly on the product.

Reference tests followed (paths in the reference repository):
``tests/test_mapper.py:53-105``, ``tests/test_fitting.py:48-90``,
``examples/fit_and_map.py:20-46``, ``tests/test_blocks.py:14-114``,
``tests/test_pipeline.py:7-62``, ``tests/test_architectures.py:66-79,126-158``.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from cachebridge_amd import layouts
from cachebridge_amd.online import peer_geometry
from cachebridge_amd.online.blocks import SourceLease, install_unpublished
from cachebridge_amd.online.pipeline import PipelinedSourceLease, layer_chunks
from oracle import install as oi
from oracle import mapper as om
from oracle.rope import apply_rope, qwen_rope

HEADWISE = torch.tensor(1, dtype=torch.int8)


def _rotated_page(seed=7, positions=range(3), scaling=None):
    torch.manual_seed(seed)
    content = torch.randn(1, 3, 2, 4)
    values = torch.randn(1, 3, 2, 4)
    cos, sin = qwen_rope(torch.tensor(list(positions)), head_dim=4, theta=10_000, scaling=scaling)
    page = torch.stack((apply_rope(content, cos, sin), values), dim=0)
    return page


def _dense_identity():
    weight = torch.zeros(8, 2, 4)
    for head in range(2):
        for dim in range(4):
            weight[head * 4 + dim, head, dim] = 1
    return {"selected": torch.tensor([0]), "k_weight": weight, "k_bias": torch.zeros(2, 4),
            "v_weight": weight.clone(), "v_bias": torch.zeros(2, 4)}


def _headwise_identity():
    weight = torch.eye(4).expand(2, 4, 4).contiguous()
    return {"selected": torch.tensor([0]), "k_weight": weight, "k_bias": torch.zeros(2, 4),
            "v_weight": weight.clone(), "v_bias": torch.zeros(2, 4), "headwise": HEADWISE}


# ----------------------------------------------------------------------------- mapper


def test_dense_identity_page():
    page = _rotated_page()
    mapper = om.PageMapper.from_tensors([_dense_identity()], method="nv_transfer",
                                        source_rope_theta=10_000, target_rope_theta=10_000)
    assert torch.allclose(mapper.map_page(page, position_start=0), page, atol=2e-6)


def test_headwise_tp_slice():
    page = _rotated_page()
    mapper = om.PageMapper.from_tensors([_headwise_identity()], method="cachebridge",
                                        source_rope_theta=10_000, target_rope_theta=10_000,
                                        target_tp_rank=1, target_tp_size=2)
    actual = mapper.map_page(page, position_start=0)
    assert actual.shape == (2, 1, 3, 1, 4)
    assert torch.allclose(actual, page[:, :, :, 1:2], atol=2e-6)


def test_headwise_yarn_identity_page():
    scaling = {"rope_type": "yarn", "factor": 2.0, "original_max_position_embeddings": 32}
    page = _rotated_page(seed=11, positions=range(40, 43), scaling=scaling)
    mapper = om.PageMapper.from_tensors([_headwise_identity()], method="cachebridge",
                                        source_rope_theta=10_000, target_rope_theta=10_000,
                                        source_rope_scaling=scaling, target_rope_scaling=scaling)
    assert torch.allclose(mapper.map_page(page, position_start=40), page, atol=2e-6)


def test_mapper_schema_errors():
    kw = dict(source_rope_theta=1e4, target_rope_theta=1e4)
    broken = _headwise_identity()
    del broken["v_bias"]
    with pytest.raises(ValueError, match="missing"):
        om.PageMapper.from_tensors([broken], method="cachebridge", **kw)
    with pytest.raises(ValueError, match="headwise"):
        om.PageMapper.from_tensors([_headwise_identity()], method="nv_transfer", **kw)
    with pytest.raises(ValueError, match="divide"):
        om.PageMapper.from_tensors([_headwise_identity()], method="cachebridge",
                                   target_tp_size=3, **kw)
    with pytest.raises(FileNotFoundError):
        om.PageMapper("/nonexistent-mapper-dir", method="cachebridge", **kw)


def _exact_affine_layer(coefficients, constant, heads, dim):
    """Head-wise layer whose map is ``sum_j a_j * src[selected_j] + c`` exactly."""
    selected = [layer for layer, _ in coefficients]
    w = torch.zeros(heads, len(selected) * dim, dim)
    for j, (_, a) in enumerate(coefficients):
        w[:, j * dim:(j + 1) * dim] = a * torch.eye(dim)
    b = torch.full((heads, dim), constant)
    return {"selected": torch.tensor(selected), "k_weight": w, "k_bias": b,
            "v_weight": w.clone(), "v_bias": b.clone(), "headwise": HEADWISE}


def test_closed_form_affine_tp_mapping():
    """``tests/test_fitting.py:48-90``: target = 0.7 src2 - 0.2 src0 + 0.13."""
    rng = torch.Generator().manual_seed(14)
    source = torch.randn(2, 3, 128, 4, 4, generator=rng)
    target = 0.7 * source[:, 2] - 0.2 * source[:, 0] + 0.13
    layer = _exact_affine_layer([(2, 0.7), (0, -0.2)], 0.13, heads=4, dim=4)
    positions = torch.arange(103, 135)
    page = source[:, :, 96:].clone()
    cos, sin = qwen_rope(positions, head_dim=4, theta=10000)
    page[0] = apply_rope(page[0], cos, sin)
    expected = target[:, None, 96:].clone()
    cos, sin = qwen_rope(positions, head_dim=4, theta=1000000)
    expected[0] = apply_rope(expected[0], cos, sin)
    before = page.clone()
    for rank in range(2):
        mapper = om.PageMapper.from_tensors([layer], method="cachebridge",
                                            source_rope_theta=10000, target_rope_theta=1000000,
                                            target_tp_size=2, target_tp_rank=rank)
        output = torch.empty(2, 1, 32, 2, 4)
        result = mapper.map_page(page, position_start=103, output=output)
        torch.testing.assert_close(result, expected[:, :, :, rank * 2:(rank + 1) * 2],
                                   atol=1e-5, rtol=1e-5)
        assert result.data_ptr() == output.data_ptr()
        compact = mapper.map_page(page[:, :, :, rank * 2:(rank + 1) * 2], position_start=103,
                                  source_head_offset=rank * 2)
        torch.testing.assert_close(compact, result, atol=0, rtol=0)
    torch.testing.assert_close(page, before, atol=0, rtol=0)


def test_closed_form_fit_and_map_example():
    """``examples/fit_and_map.py:20-46``: target = 0.6 src0 + 0.3 src2 + 0.1, aliased output."""
    rng = torch.Generator().manual_seed(42)
    source = torch.randn(2, 3, 256, 2, 4, generator=rng)
    target = 0.6 * source[:, 0] + 0.3 * source[:, 2] + 0.1
    layer = _exact_affine_layer([(0, 0.6), (2, 0.3)], 0.1, heads=2, dim=4)
    mapper = om.PageMapper.from_tensors([layer], method="cachebridge", source_rope_theta=10000,
                                        target_rope_theta=1000000)
    page = source[:, :, 192:].clone()
    positions = torch.arange(192, 256)
    cos, sin = qwen_rope(positions, head_dim=4, theta=10000)
    page[0] = apply_rope(page[0], cos, sin)
    output = torch.empty(2, 1, 64, 2, 4)
    result = mapper.map_page(page, position_start=192, output=output)
    expected = target[:, None, 192:].clone()
    cos, sin = qwen_rope(positions, head_dim=4, theta=1000000)
    expected[0] = apply_rope(expected[0], cos, sin)
    torch.testing.assert_close(result, expected, atol=1e-5, rtol=1e-5)
    assert result.data_ptr() == output.data_ptr()


# ----------------------------------------------------------------------------- blocks


def test_source_cannot_reuse_or_release_before_gpu_ack():
    events = []
    lease = SourceLease(lambda: events.append("lock"), lambda: events.append("unlock"))
    lease.begin()
    lease.export(0, 512)
    with pytest.raises(RuntimeError):
        lease.export(512, 513)
    with pytest.raises(RuntimeError):
        lease.close()
    with pytest.raises(RuntimeError):
        lease.acknowledge(gpu_reads_complete=False)
    lease.acknowledge(gpu_reads_complete=True)
    lease.export(512, 513)
    lease.acknowledge(gpu_reads_complete=True)
    lease.close()
    assert events == ["lock", "unlock"]


def test_oracle_gather_partial_block_noncontiguous_pages():
    k = torch.arange(3 * 700 * 2 * 4).reshape(3, 700, 2, 4).float()
    v = -k
    pool = SimpleNamespace(layer_num=3, start_layer=0, _get_key_buffer=lambda l: k[l],
                           _get_value_buffer=lambda l: v[l])
    indices = torch.randperm(650, generator=torch.Generator().manual_seed(7))[:513] + 1
    workspace = torch.empty(2 * 3 * 512 * 2 * 4)
    for start, stop in [(0, 65), (0, 512), (512, 513)]:
        packed = oi.pack_source_block(pool, indices, start=start, stop=stop,
                                      workspace=workspace, block_tokens=512)
        assert packed.is_contiguous() and packed.data_ptr() == workspace.data_ptr()
        expected = torch.stack([torch.stack([k[l, indices[start:stop]], v[l, indices[start:stop]]])
                                for l in range(3)], dim=1)
        assert torch.equal(packed, expected)


def _transaction(*, foreign_failure=False, cancel=None, broken_span=False):
    events = []
    value = torch.zeros(2, 1, 2, 1, 1)
    blocks = [(0, 2, value), (3 if broken_span else 2, 4, value)]
    kwargs = dict(
        token_count=4,
        allocate=lambda n: torch.tensor([5, 2, 9, 3]),
        free=lambda indices: events.append(("free", indices.tolist())),
        blocks=blocks,
        write=lambda value, indices, start: events.append(("write", start)),
        synchronize=lambda: events.append(("sync",)),
        ready_vote=lambda local: events.append(("vote", local)) or (local and not foreign_failure),
        publish=lambda indices: events.append(("publish", indices.tolist())),
        cancel_after_blocks=cancel,
    )
    return events, kwargs


def test_publish_only_after_complete_writes_and_ready_vote():
    events, kwargs = _transaction()
    assert install_unpublished(**kwargs)["published"]
    assert events[-2][0] == "vote" and events[-1][0] == "publish"
    assert "free" not in [e[0] for e in events]


@pytest.mark.parametrize("options", [dict(cancel=1), dict(foreign_failure=True),
                                     dict(broken_span=True)])
def test_cancellation_or_foreign_failure_frees_unpublished_once(options):
    events, kwargs = _transaction(**options)
    with pytest.raises(RuntimeError, match="rolled back"):
        install_unpublished(**kwargs)
    assert [e[0] for e in events].count("free") == 1
    assert "publish" not in [e[0] for e in events]


def test_broken_vote_does_not_claim_safe_global_reclamation():
    events, kwargs = _transaction()

    def fail(_):
        raise RuntimeError("distributed group unavailable")

    kwargs["ready_vote"] = fail
    with pytest.raises(RuntimeError, match="distributed group"):
        install_unpublished(**kwargs)
    assert "free" not in [e[0] for e in events]


# ----------------------------------------------------------------------------- pipeline


def test_two_live_slots_require_individual_completion():
    events = []
    lease = PipelinedSourceLease(lambda: events.append("acquire"),
                                 lambda: events.append("release"))
    lease.begin()
    lease.export(0, 0, 2048)
    lease.export(1, 2048, 4096)
    with pytest.raises(RuntimeError):
        lease.export(0, 4096, 4097)
    with pytest.raises(RuntimeError):
        lease.close()
    with pytest.raises(RuntimeError):
        lease.acknowledge(0, gpu_reads_complete=False)
    lease.acknowledge(0, gpu_reads_complete=True)
    lease.export(0, 4096, 4097)
    lease.acknowledge(1, gpu_reads_complete=True)
    with pytest.raises(RuntimeError):
        lease.close()
    lease.acknowledge(0, gpu_reads_complete=True)
    lease.close()
    assert events == ["acquire", "release"]


@pytest.mark.parametrize("tokens", [1, 512, 2048, 4096])
def test_peer_geometry_covers_fragmented_destination_without_overlap(tokens):
    split = max(1, tokens // 2)
    runs = [(0, split, 5)]
    if split < tokens:
        runs.append((split, tokens, split + 20))
    row_bytes = 2 * 128 * 2
    copies = peer_geometry.operations(0, tokens, runs, heads=2)
    assert sum(size for *_, size in copies) == 2 * 64 * tokens * row_bytes
    for kind in range(2):
        for layer in range(64):
            spans = [(src, dst, size) for k, l, src, dst, size in copies if (k, l) == (kind, layer)]
            cursor = (kind * 64 + layer) * tokens * row_bytes
            for (a, b, physical), (src, dst, size) in zip(runs, spans):
                assert src == cursor
                assert dst == physical * row_bytes
                assert size == (b - a) * row_bytes
                cursor += size
            assert cursor == (kind * 64 + layer + 1) * tokens * row_bytes


def test_peer_geometry_rejects_alias_and_unsupported_block():
    with pytest.raises(ValueError, match="alias"):
        peer_geometry.operations(0, 8, [(0, 4, 5), (4, 8, 7)], heads=2)
    with pytest.raises(ValueError, match="unsupported"):
        peer_geometry.operations(0, 4097, [(0, 4097, 0)], heads=2)
    with pytest.raises(ValueError, match="partition"):
        peer_geometry.operations(0, 8, [(0, 4, 0), (5, 8, 100)], heads=2)
    with pytest.raises(ValueError, match="cover"):
        peer_geometry.operations(0, 8, [(0, 4, 0)], heads=2)


def test_contiguous_runs_and_slots_round_trip():
    g = torch.Generator().manual_seed(9)
    pages = torch.randperm(64, generator=g)[:20]
    slots = (pages[:, None] * 16 + torch.arange(16)).reshape(-1)[:300]
    runs = peer_geometry.contiguous_runs(slots)
    assert runs[0][0] == 0 and runs[-1][1] == 300
    assert all(a[1] == b[0] for a, b in zip(runs, runs[1:]))
    assert torch.equal(peer_geometry.slots_from_runs(runs, 0, 300), slots.long())
    assert torch.equal(peer_geometry.slots_from_runs(runs, 17, 211), slots[17:211].long())
    assert peer_geometry.contiguous_runs([]) == []
    assert peer_geometry.contiguous_runs([4, 5, 6, 9]) == [(0, 3, 4), (3, 4, 9)]


# ----------------------------------------------------------------------------- layouts


def test_head_ownership_requires_explicit_mapping_for_different_counts():
    assert layouts.head_assignment(2, 2) == (0, 1)
    with pytest.raises(ValueError, match="explicit"):
        layouts.head_assignment(2, 4)
    assert layouts.head_assignment(2, 4, [0, 0, 1, 1]) == (0, 0, 1, 1)
    with pytest.raises(ValueError, match="valid source head"):
        layouts.head_assignment(2, 4, [0, 0, 1, 2])


def test_gemma_implicit_layer_pattern():
    assert layouts.gemma_layer_types(6) == [layouts.SLIDING] * 5 + [layouts.FULL]
    kinds = layouts.gemma_layer_types(62)
    assert [i for i, k in enumerate(kinds) if k == layouts.FULL] == list(range(5, 62, 6))


def test_gemma_window_keeps_last_window_minus_one_tokens():
    """``tests/test_architectures.py:126-144``: W=4 keeps 3 of 9 tokens, first position 6."""
    assert layouts.retained_window(9, layer_type=layouts.SLIDING, sliding_window=4) == (6, 3)
    assert layouts.retained_window(9, layer_type=layouts.FULL) == (0, 9)
    assert layouts.retained_window(2, layer_type=layouts.SLIDING, sliding_window=4) == (0, 2)
    assert oi.materialize_window(9, layer_type="sliding_attention", sliding_window=4) == 6
    with pytest.raises(ValueError, match="room"):
        layouts.retained_window(9, layer_type=layouts.SLIDING, sliding_window=1)
    with pytest.raises(ValueError, match="Unsupported"):
        layouts.retained_window(9, layer_type="linear_attention")
    assert layouts.mapper_windows(layouts.gemma_layer_types(6), 1024) == [1024] * 5 + [None]


def test_layer_chunks_never_mix_window_classes():
    windows = layouts.mapper_windows(layouts.gemma_layer_types(62), 1024)
    chunks = layer_chunks(windows, 4)
    assert sorted(l for c in chunks for l in c) == list(range(62))
    assert all(len(c) <= 4 and len({windows[l] for l in c}) == 1 for c in chunks)
    assert len(chunks) == 3 + 13  # 10 full layers -> 3 chunks, 52 local -> 13
