"""Checks shared by the GPU tests that run the configured workloads at full size.

A full-size launch is checked without a full-size oracle run:

- every target pool is first filled with a sentinel bit pattern (a bf16 NaN
  with a payload, which no mapped value takes), so "every row outside the
  request's slots and windows is bit-unchanged" is a scan on the GPU: those
  rows still hold the sentinel, and every written row no longer does;
- the rows at the request's target slots are snapshot after one launch and
  compared bit for bit with a second run of the same work split differently
  (block by block, or request by request);
- the oracle maps sampled token windows (first, middle and last 64 tokens, and
  both sides of each sliding-window edge) for sampled target layers, all heads,
  K and V, from the same source rows read back from the pool; the GPU rows at
  those tokens' slots must match it to the parity bar of
  ``oracle.tolerance.check_mapped``.
"""

from __future__ import annotations

import torch

from oracle import install as oi
from oracle import tolerance as ot

SENTINEL = 0x7FBF  # int16 view of a bf16 quiet NaN with a payload


def fill_sentinel(pool) -> None:
    pool.k_data.view(torch.int16).fill_(SENTINEL)
    pool.v_data.view(torch.int16).fill_(SENTINEL)


def first_kept(windows, layers: int, prefix: int, position_start: int = 0) -> list[int]:
    """Request-local index of the first token each target layer keeps."""
    out = []
    for l in range(layers):
        w = None if windows is None else windows[l]
        first_pos = 0 if w is None else oi.materialize_window(prefix, layer_type="sliding_attention",
                                                              sliding_window=w)
        out.append(max(0, first_pos - position_start))
    return out


def check_untouched(pool, written: list[torch.Tensor]) -> None:
    """Rows outside ``written[l]`` (device int64 row indices per layer) hold the sentinel.

    Every row in ``written[l]`` must no longer hold it (the launch wrote it).
    """
    dev = pool.k_data.device
    for kind, bufs in ((0, pool.k_buffer), (1, pool.v_buffer)):
        for l, buf in enumerate(bufs):
            mask = torch.zeros(buf.shape[0], dtype=torch.bool, device=dev)
            mask[written[l]] = True
            sent = (buf.view(torch.int16) == SENTINEL).flatten(1).all(1)
            assert bool(sent[~mask].all()), f"kind {kind} layer {l}: a row outside the request changed"
            assert not bool(sent[mask].any()), f"kind {kind} layer {l}: a request row was not written"


def snapshot(pool, slots: torch.Tensor) -> torch.Tensor:
    """``[2, layers, n, heads, D]`` int16 bit patterns of the rows at ``slots`` (device).

    Bit patterns, so that sentinel NaNs (tokens outside a window) compare equal.
    """
    return torch.stack([torch.stack([b[slots] for b in pool.k_buffer]),
                        torch.stack([b[slots] for b in pool.v_buffer])]).view(torch.int16)


def token_windows(n: int, width: int = 64, edges=()) -> list[tuple[int, int]]:
    """First, middle and last ``width`` tokens of ``n``, plus ``width`` tokens centred on each edge."""
    spans = {(0, min(width, n)), (max(0, n // 2 - width // 2), min(n, n // 2 + width // 2)),
             (max(0, n - width), n)}
    for e in edges:
        if 0 < e < n:
            spans.add((max(0, e - width // 2), min(n, e + width // 2)))
    return sorted(spans)


def oracle_window(source_pool, src_slots: torch.Tensor, target_pool, tgt_slots: torch.Tensor,
                  spec: dict, *, lo: int, hi: int, position_start: int, layers: list[int],
                  source_theta: float, target_thetas, first: list[int]) -> list[dict]:
    """Compare tokens ``[lo, hi)`` of one request with the oracle for ``layers``.

    ``src_slots`` / ``tgt_slots`` are the request's per-token source and target
    rows (token order); ``first[l]`` is layer ``l``'s first kept token (rows of
    earlier tokens must still hold the sentinel). Returns the tolerance
    statistics of each (theta group) comparison.
    """
    lt = spec["assign_layer"].shape[0]
    thetas = [target_thetas] * lt if isinstance(target_thetas, (int, float)) else list(target_thetas)
    s_rows = src_slots[lo:hi].long()
    t_rows = tgt_slots[lo:hi].long()
    page = torch.stack([
        torch.stack([source_pool._get_key_buffer(l)[s_rows] for l in range(source_pool.layer_num)]),
        torch.stack([source_pool._get_value_buffer(l)[s_rows] for l in range(source_pool.layer_num)]),
    ]).cpu()
    virtual = oi.virtual_source_page(page, spec["assign_layer"], spec["assign_head"])
    stats = []
    for theta in sorted({thetas[l] for l in layers}):
        group = [l for l in layers if thetas[l] == theta]
        mapper = oi.assignment_mapper(spec, group, source_rope_theta=source_theta,
                                      target_rope_theta=theta)
        ref = mapper.map_page(virtual, position_start=position_start + lo)
        got = torch.stack([
            torch.stack([target_pool.k_buffer[l][t_rows] for l in group]),
            torch.stack([target_pool.v_buffer[l][t_rows] for l in group]),
        ]).cpu()
        sub = {k: spec[k][group] for k in ("assign_layer", "assign_head", "k_weight", "v_weight",
                                            "k_bias", "v_bias")}
        bound = ot.magnitude_bound(page, sub, position_start=position_start + lo,
                                   source_theta=source_theta, target_thetas=[theta] * len(group))
        for i, l in enumerate(group):
            keep = min(max(first[l] - lo, 0), hi - lo)  # tokens before the layer's window
            if keep:
                untouched = got[:, i, :keep].contiguous().view(torch.int16)
                assert bool((untouched == SENTINEL).all()), f"layer {l}: a token before the window was written"
            if keep < hi - lo:
                st = ot.check_mapped(got[:, i, keep:], ref[:, i, keep:], bound[:, i, keep:])
                st.update(layer=l, tokens=(lo + keep, hi))
                stats.append(st)
    return stats


def summarize(stats: list[dict]) -> dict:
    """Worst-case figures over many ``check_mapped`` results."""
    elems = sum(s["elements"] for s in stats)
    within = sum(s["within_1ulp"] * s["elements"] for s in stats) / max(elems, 1)
    return {"checks": len(stats), "elements": elems, "within_1ulp": within,
            "beyond_1ulp_fraction": 1.0 - within,
            "max_ulp": max((s["max_ulp"] for s in stats), default=0),
            "max_rel_norm": max((s["rel_norm"] for s in stats), default=0.0),
            "max_rel_elem": max((s["max_rel_elem"] for s in stats), default=0.0),
            "rel_elem_fraction": (sum(s["rel_elem_fraction"] * s["elements"] for s in stats)
                                  / max(elems, 1))}
