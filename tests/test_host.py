"""Host logic without a device: workload shapes, byte accounting, row descriptors, bench CLI."""

from __future__ import annotations

import subprocess
import sys

import pytest
import torch

from cachebridge_amd import synthetic
from cachebridge_amd.plan import rows_from_page, rows_from_stacked

from .conftest import ROOT


def _distinct_pairs(sh):
    spec = synthetic.mapper_spec(sh)
    return len({(int(l), int(h)) for l, h in zip(spec["assign_layer"].flatten(),
                                                  spec["assign_head"].flatten())})


@pytest.mark.parametrize("name,expected", [("tp4", 350_388_224), ("full", 1_407_746_048)])
def test_algorithmic_bytes_closed_form(name, expected):
    """B = target writes + distinct source pairs read once + fp32 maps once + token index."""
    sh = synthetic.shape(name)
    lt, ht, d, t = sh.target_layers, sh.target_heads, sh.head_dim, sh.tokens
    pairs = _distinct_pairs(sh)
    closed = 2 * 2 * d * lt * ht * t + 2 * 2 * d * pairs * t + 4 * 2 * lt * ht * (d * d + d) + 8 * t
    assert synthetic.algorithmic_bytes(sh) == closed == expected
    # Every target head draws its source from the 16 evenly spaced selected layers.
    assert synthetic.mapper_spec(sh)["selected"] == [round(x) for x in
                                                    torch.linspace(0, 39, 16).tolist()]


def test_gemma_shape_windows_and_bytes():
    sh = synthetic.shape("gemma")
    full = [l for l in range(62) if sh.windows[l] is None]
    assert full == list(range(5, 62, 6))
    assert [synthetic.window_tokens(sh, l) for l in (0, 5)] == [1023, 8192]
    spec = synthetic.mapper_spec(sh)
    assert torch.equal(spec["assign_head"][0, :, 0], torch.arange(16) // 2)
    tokens = 10 * 8192 + 52 * 1023
    assert synthetic.algorithmic_flops(sh) == 2 * 2 * tokens * 16 * 128 * 128


def test_toy_shape_is_fp32_with_four_selected_layers():
    sh = synthetic.shape("toy")
    spec = synthetic.mapper_spec(sh)
    assert sh.dtype == torch.float32 and len(spec["selected"]) == 4
    assert set(spec["assign_layer"].unique().tolist()) <= set(spec["selected"])
    with pytest.raises(ValueError, match="unknown"):
        synthetic.shape("nope")


def test_slots_follow_the_block_table():
    pages = synthetic.fragmented_pages(64, 10, seed=3)
    assert len(set(pages.tolist())) == 10 and int(pages.max()) < 64
    slots = synthetic.slots_from_pages(pages, 150, 16)
    t = torch.arange(150)
    assert torch.equal(slots, pages.long()[t // 16] * 16 + t % 16)
    with pytest.raises(ValueError):
        synthetic.fragmented_pages(4, 5, seed=0)


def test_row_descriptors_describe_strides_and_indices():
    page = torch.zeros(2, 3, 10, 2, 8, dtype=torch.bfloat16)
    r = rows_from_page(page, head_offset=1)
    assert (r.c.num_layers, r.c.rows, r.c.heads, r.c.head_offset) == (3, 10, 2, 1)
    assert r.c.layer_stride == 10 * 2 * 8 and r.c.row_stride == 16
    assert r.c.k_base == page[0].data_ptr() and r.c.v_base == page[1].data_ptr()
    k = torch.zeros(4, 64, 2, 8, dtype=torch.bfloat16)
    bt = torch.tensor([3, 1], dtype=torch.int32)
    r = rows_from_stacked(k, k.clone(), block_table=bt, page_size=16, tokens=32)
    assert r.c.index == bt.data_ptr() and r.c.page_size == 16 and r.c.rows == 64
    with pytest.raises(ValueError, match="cover"):
        rows_from_stacked(k, k.clone(), block_table=bt, page_size=16, tokens=33)
    with pytest.raises(ValueError, match="either"):
        rows_from_stacked(k, k.clone(), block_table=bt, index=bt.long(), page_size=16)
    with pytest.raises(ValueError, match="int32"):
        rows_from_stacked(k, k.clone(), block_table=bt.long(), page_size=16)
    with pytest.raises(ValueError, match="contiguous"):
        rows_from_page(page.transpose(2, 3))


def test_bench_refuses_more_than_one_gpu():
    out = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 2
    assert "one GPU" in out.stderr


def test_bench_traffic_is_used_only_for_the_kernel_source_it_was_measured_on(tmp_path, monkeypatch):
    import importlib.util
    import re

    spec = importlib.util.spec_from_file_location("bench_module", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    now = bench.kernel_source_sha16()
    for workload in ("tp4", "full"):
        traffic, source = bench.profiled_traffic("map_install_stream", workload)
        text = (ROOT / "profiles" / f"map_install_stream_{workload}_traffic.md").read_text()
        if f"kernel_source_sha16 = {now}" in text:
            assert isinstance(traffic, int) and f"traffic_bytes_per_launch = {traffic}" in text
            assert "not measured in this run" in source
        else:
            assert traffic is None and "not used" in source
    assert bench.profiled_traffic("map_install_stream", "no_such_workload") == (None, "not measured")
    # a summary of the current source is used, one of another source is not
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    (tmp_path / "profiles").mkdir()
    f = tmp_path / "profiles" / "k_w_traffic.md"
    f.write_text(f"traffic_bytes_per_launch = 123\nkernel_source_sha16 = {now}\nmeasured = today\n")
    assert bench.profiled_traffic("k", "w")[0] == 123
    f.write_text("traffic_bytes_per_launch = 123\nkernel_source_sha16 = 0000000000000000\n")
    assert bench.profiled_traffic("k", "w")[0] is None
    # every profile summary the design notes point to is committed
    design = (ROOT / "DESIGN.md").read_text()
    named = set(re.findall(r"profiles/([A-Za-z0-9_]+\.md)", design))
    assert named and all((ROOT / "profiles" / n).exists() for n in named), sorted(named)


def test_ragged_batch_lengths_and_bytes():
    lengths = synthetic.request_lengths()
    assert len(lengths) == 64 and sum(lengths) == 137_440
    assert all(256 <= n <= 16384 for n in lengths)
    assert synthetic.request_lengths() == lengths  # seeded
    clipped = synthetic.request_lengths(count=2000, sigma=2.0)
    assert min(clipped) == 256 and max(clipped) == 16384
    for name, heads in (("batch", 2), ("batch_full", 8)):
        sh = synthetic.shape(name)
        assert (sh.target_heads, sh.tokens) == (heads, 137_440)
        pairs = _distinct_pairs(sh)
        t, d = sh.tokens, sh.head_dim
        closed = (2 * 2 * d * 64 * heads * t + 2 * 2 * d * pairs * t
                  + 4 * 2 * 64 * heads * (d * d + d) + 8 * t)
        assert synthetic.algorithmic_bytes(sh) == closed


def test_request_span_defaults():
    from cachebridge_amd.plan import RequestSpan, _span_array

    sp = RequestSpan(10, 32, 5)
    assert (sp.position_start, sp.prefix_length) == (0, 0)
    arr = _span_array([sp, (0, 0, 0, 7, 9)])
    assert (arr[0].source_offset, arr[0].target_offset, arr[0].num_tokens) == (10, 32, 5)
    assert (arr[1].position_start, arr[1].prefix_length, arr[1].reserved) == (7, 9, 0)
