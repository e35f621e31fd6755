"""MI355X ``PageMapper``: the reference mapper API on the fused HIP handoff kernel.

``PageMapper(mapper_dir, *, method, source_rope_theta, target_rope_theta, ...)``
keeps the reference constructor (``cb/mapper.py:35-110``: sorted
``layer_*.safetensors``, schema check, TP head slice) and ``map_page``
contract (``cb/mapper.py:117-239``: ``[2, layers, tokens, kv_heads,
head_dim]`` in and out, output dtype = source dtype, preallocated ``output``
returned aliased, input never mutated, ``ValueError`` on geometry mismatch).
The computation runs entirely in ``libcachebridge_hip``; there is no CPU path.

Beyond the reference file format, ``HeadwiseMapper.from_assignment`` accepts
an arbitrary source ``(layer, head)`` list per target ``(layer, head)``, per
target layer RoPE theta and sliding-window class (Gemma 3 local/global
layouts, ``cb/architectures/gemma3.py:39-58``).
"""

from __future__ import annotations

from pathlib import Path
from typing import Sequence

import numpy as np
import torch

from . import _lib
from .plan import HandoffPlan, RequestSpan, Rows, ThetaSet, rows_from_page


class HeadwiseMapper:
    """Head-wise affine KV mapper bound to one GPU.

    ``assign_layer``/``assign_head``: ``[Lt, Ht, s]`` global source indices per
    local target (layer, head); ``k_weight``/``v_weight``: ``[Lt, Ht, s*D, D]``
    fp32 (``y = x @ W``); ``k_bias``/``v_bias``: ``[Lt, Ht, D]``.
    ``target_rope_theta``/``target_rope_scaling`` may be per target layer;
    ``windows`` is a per-target-layer list of ``None`` (keep all tokens) or a
    sliding window size ``W`` (keep the last ``min(prefix, W-1)`` tokens).
    """

    method = "cachebridge"

    def _init_plan(self, *, assign_layer, assign_head, k_weight, k_bias, v_weight, v_bias,
                   source_rope_theta, target_rope_theta, source_rope_scaling=None,
                   target_rope_scaling=None, windows=None, dtype=torch.bfloat16, device="cuda",
                   max_positions: int = 40960, target_head_start: int = 0,
                   target_head_stop: int | None = None) -> None:
        al = torch.as_tensor(assign_layer, dtype=torch.int64).cpu()
        ah = torch.as_tensor(assign_head, dtype=torch.int64).cpu()
        if al.ndim != 3 or al.shape != ah.shape:
            raise ValueError("assign_layer/assign_head must be matching [layers, heads, support]")
        lt, ht, s = al.shape
        d = int(k_weight.shape[-1])
        for name, t, shape in (("k_weight", k_weight, (lt, ht, s * d, d)),
                               ("v_weight", v_weight, (lt, ht, s * d, d)),
                               ("k_bias", k_bias, (lt, ht, d)), ("v_bias", v_bias, (lt, ht, d))):
            if tuple(t.shape) != shape:
                raise ValueError(f"{name} must be {shape}, got {tuple(t.shape)}")
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("HeadwiseMapper runs on a GPU device; there is no CPU path")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.dtype = dtype
        self.head_dim = d
        self.support = s
        self.assign_layer, self.assign_head = al, ah
        self.target_head_start = int(target_head_start)
        self.target_head_stop = int(target_head_stop if target_head_stop is not None
                                    else target_head_start + ht)
        self.local_heads = ht
        self.source_rope_theta = float(source_rope_theta)
        self.source_rope_scaling = source_rope_scaling
        per_layer_theta = (list(target_rope_theta) if isinstance(target_rope_theta, (list, tuple))
                           else [target_rope_theta] * lt)
        per_layer_scaling = (list(target_rope_scaling) if isinstance(target_rope_scaling, (list, tuple))
                             else [target_rope_scaling] * lt)
        if len(per_layer_theta) != lt or len(per_layer_scaling) != lt:
            raise ValueError("per-layer target RoPE settings need one entry per target layer")
        self.target_rope_theta = target_rope_theta
        self.target_rope_scaling = target_rope_scaling
        windows = list(windows) if windows is not None else [None] * lt
        if len(windows) != lt:
            raise ValueError("windows needs one entry per target layer")
        self.windows = windows
        theta_sets: list[ThetaSet] = []

        def theta_index(ts: ThetaSet) -> int:
            for i, known in enumerate(theta_sets):
                if known.key() == ts.key():
                    return i
            theta_sets.append(ts)
            return len(theta_sets) - 1

        src_theta = theta_index(ThetaSet(self.source_rope_theta, source_rope_scaling))
        layer_theta = [theta_index(ThetaSet(float(t), sc))
                       for t, sc in zip(per_layer_theta, per_layer_scaling)]
        window_sizes = sorted({0 if w is None else int(w) for w in windows})
        layer_window = [window_sizes.index(0 if w is None else int(w)) for w in windows]

        jobs = lt * ht * 2
        tl = np.repeat(np.arange(lt), ht * 2)
        th = np.tile(np.repeat(np.arange(ht), 2), lt)
        kind = np.tile(np.array([_lib.CB_KIND_K, _lib.CB_KIND_V]), lt * ht)
        src_l = np.repeat(al.reshape(lt * ht, s).numpy(), 2, axis=0)
        src_h = np.repeat(ah.reshape(lt * ht, s).numpy(), 2, axis=0)
        w = torch.stack((torch.as_tensor(k_weight), torch.as_tensor(v_weight)), dim=2)
        b = torch.stack((torch.as_tensor(k_bias), torch.as_tensor(v_bias)), dim=2)
        self._jobs = {
            "job_target_layer": tl, "job_target_head": th, "job_kind": kind,
            "source_layers": src_l, "source_heads": src_h,
            "weights": w.reshape(jobs, s * d, d), "biases": b.reshape(jobs, d),
            "job_source_theta": np.full(jobs, src_theta),
            "job_target_theta": np.repeat(np.asarray(layer_theta), ht * 2),
            "job_window": np.repeat(np.asarray(layer_window), ht * 2),
        }
        self._theta_sets = theta_sets
        self._window_sizes = window_sizes
        self._max_positions = int(max_positions)
        self.plan = HandoffPlan(
            head_dim=d, dtype=dtype, target_layers=lt, target_heads=ht, thetas=theta_sets,
            window_sizes=window_sizes, max_positions=max_positions, device=self.device,
            **self._jobs,
        )
        self._target_layers = lt
        self._max_source_layer = int(al.max())
        self._source_heads = (int(ah.min()), int(ah.max()))
        self._source_layers = tuple(sorted({int(x) for x in al.flatten().tolist()}))

    @classmethod
    def from_assignment(cls, **kwargs) -> "HeadwiseMapper":
        self = cls.__new__(cls)
        self._init_plan(**kwargs)
        return self

    @property
    def source_layers(self) -> tuple:
        """Source layers any job reads (the layers a receiver must be sent)."""
        return self._source_layers

    @property
    def target_layers(self) -> int:
        return self._target_layers

    def layer_plan(self, layers: Sequence[int]) -> HandoffPlan:
        """A plan for a subset of target layers; its target layer ``i`` is ``layers[i]``.

        Same maps, RoPE settings and window classes as the full plan, so every
        mapped row is bit-identical to the full plan's (used by the staged
        layer-chunk pipeline).
        """
        layers = [int(l) for l in layers]
        if not layers or len(set(layers)) != len(layers) or not all(
                0 <= l < self._target_layers for l in layers):
            raise ValueError("layer_plan needs distinct target layers of this mapper")
        tl = self._jobs["job_target_layer"]
        pick = np.concatenate([np.flatnonzero(tl == l) for l in layers])
        local = np.empty(self._target_layers, dtype=np.int64)
        local[layers] = np.arange(len(layers))
        sub = {k: (v[torch.as_tensor(pick)] if isinstance(v, torch.Tensor) else v[pick])
               for k, v in self._jobs.items()}
        sub["job_target_layer"] = local[tl[pick]]
        return HandoffPlan(
            head_dim=self.head_dim, dtype=self.dtype, target_layers=len(layers),
            target_heads=self.local_heads, thetas=self._theta_sets,
            window_sizes=self._window_sizes, max_positions=self._max_positions,
            device=self.device, **sub,
        )

    def _check_positions(self, position_start: int, tokens: int) -> None:
        if position_start < 0 or position_start + tokens > self.plan.max_positions:
            raise ValueError(
                f"positions [{position_start}, {position_start + tokens}) exceed the plan's "
                f"RoPE table of {self.plan.max_positions} positions"
            )

    def _check_source_heads(self, offset: int, heads: int) -> None:
        lo, hi = self._source_heads
        if lo - offset < 0 or hi - offset >= heads:
            raise ValueError("CacheBridge source-head geometry mismatch")

    @torch.inference_mode()
    def map_page(self, source_page: torch.Tensor, *, position_start: int,
                 source_head_offset: int = 0, output_device="cpu",
                 output: torch.Tensor | None = None) -> torch.Tensor:
        """Map one ``[2, Ls, n, Hs, D]`` page to ``[2, Lt, n, Ht, D]`` (``cb/mapper.py:117-239``)."""
        if source_page.ndim != 5 or source_page.shape[0] != 2:
            raise ValueError("source page must be [2,layers,tokens,kv_heads,head_dim]")
        page = source_page.to(self.device)
        if page.dtype != self.dtype:
            raise ValueError(f"source page dtype {page.dtype} differs from the mapper's {self.dtype}")
        if not page.is_contiguous():
            page = page.contiguous()
        _, depth, tokens, heads, dim = page.shape
        if dim != self.head_dim:
            raise ValueError("CacheBridge source-head geometry mismatch")
        if self._max_source_layer >= depth:
            raise ValueError("mapper selected layer exceeds source page depth")
        self._check_source_heads(source_head_offset, heads)
        self._check_positions(position_start, tokens)
        expected = (2, self.target_layers, tokens, self.local_heads, dim)
        want = torch.device(output_device)
        if want.type == "cuda" and want.index is None:
            want = torch.device("cuda", torch.cuda.current_device())
        if output is not None:
            if (tuple(output.shape) != expected or output.dtype != self.dtype
                    or output.device != want):
                raise ValueError("preallocated mapper output geometry/dtype/device mismatch")
        direct = output is not None and output.device == self.device and output.is_contiguous()
        out = output if direct else torch.empty(expected, dtype=self.dtype, device=self.device)
        if any(w is not None for w in self.windows):
            # Window-excluded tokens of a dense output are not computed; define them.
            out.zero_()
        self.plan.launch(rows_from_page(page, head_offset=source_head_offset), rows_from_page(out),
                         num_tokens=tokens, position_start=position_start)
        if output is None:
            return out.to(output_device)
        if not direct:
            output.copy_(out)
        return output

    def map_install(self, source: Rows, target: Rows, *, num_tokens: int, position_start: int,
                    prefix_length: int = 0, stream: torch.cuda.Stream | None = None,
                    tokens_per_workgroup: int = 0) -> None:
        """Fused gather -> map -> install of one block (asynchronous on ``stream``).

        ``source``/``target`` describe K/V buffers and token -> row indices
        (``cachebridge_amd.plan.rows_from_*``); token ``t`` of the block sits
        at position ``position_start + t``.
        """
        if source.num_layers <= self._max_source_layer:
            raise ValueError("mapper selected layer exceeds source depth")
        self._check_source_heads(source.c.head_offset, source.c.heads)
        self._check_positions(position_start, num_tokens)
        self.plan.launch(source, target, num_tokens=num_tokens, position_start=position_start,
                         prefix_length=prefix_length, stream=stream,
                         tokens_per_workgroup=tokens_per_workgroup)

    def map_install_batch(self, source: Rows, target: Rows, spans, *,
                          stream: torch.cuda.Stream | None = None) -> None:
        """Fused gather -> map -> install of many requests in one launch (asynchronous).

        ``spans`` are ``plan.RequestSpan`` tuples over the shared ``source`` /
        ``target`` descriptions; every row a request writes equals what
        ``map_install`` writes for that request alone.
        """
        if source.num_layers <= self._max_source_layer:
            raise ValueError("mapper selected layer exceeds source depth")
        self._check_source_heads(source.c.head_offset, source.c.heads)
        for sp in spans:
            sp = RequestSpan(*sp)
            if sp.num_tokens < 0:
                raise ValueError("a request cannot have a negative token count")
            self._check_positions(sp.position_start, sp.num_tokens)
        self.plan.launch_batch(source, target, spans, stream=stream)


class PageMapper(HeadwiseMapper):
    """Reference-compatible constructor over ``layer_*.safetensors`` (``cb/mapper.py:35-110``)."""

    def __init__(self, mapper_dir, *, method: str, source_rope_theta: float,
                 target_rope_theta: float, source_rope_scaling: dict | None = None,
                 target_rope_scaling: dict | None = None, device="cuda",
                 target_tp_rank: int = 0, target_tp_size: int = 1,
                 dtype: torch.dtype = torch.bfloat16, max_positions: int = 40960) -> None:
        from safetensors.torch import load_file

        if method != "cachebridge":
            raise ValueError(
                f"method={method!r}: only head-wise CacheBridge maps run on the MI355X path "
                "(the dense nv_transfer regression mode is not supported)"
            )
        self.mapper_dir = Path(mapper_dir)
        self.target_tp_rank = int(target_tp_rank)
        self.target_tp_size = int(target_tp_size)
        paths = sorted(self.mapper_dir.glob("layer_*.safetensors"))
        if not paths:
            raise FileNotFoundError(f"no layer_*.safetensors in {self.mapper_dir}")
        self.layers = [load_file(str(p)) for p in paths]
        self._build_from_layers([str(p) for p in paths], source_rope_theta, target_rope_theta,
                                source_rope_scaling, target_rope_scaling, device, dtype,
                                max_positions)

    @classmethod
    def from_tensors(cls, layers: Sequence[dict], *, method: str = "cachebridge",
                     source_rope_theta: float, target_rope_theta: float,
                     source_rope_scaling=None, target_rope_scaling=None, device="cuda",
                     target_tp_rank: int = 0, target_tp_size: int = 1,
                     dtype: torch.dtype = torch.bfloat16, max_positions: int = 40960) -> "PageMapper":
        """Build from in-memory ``layer_*.safetensors`` dictionaries (same checks)."""
        if method != "cachebridge":
            raise ValueError("only head-wise CacheBridge maps run on the MI355X path")
        self = cls.__new__(cls)
        self.mapper_dir = None
        self.target_tp_rank = int(target_tp_rank)
        self.target_tp_size = int(target_tp_size)
        self.layers = list(layers)
        self._build_from_layers([f"layer {i}" for i in range(len(self.layers))], source_rope_theta,
                                target_rope_theta, source_rope_scaling, target_rope_scaling,
                                device, dtype, max_positions)
        return self

    def _build_from_layers(self, names, source_rope_theta, target_rope_theta,
                           source_rope_scaling, target_rope_scaling, device, dtype,
                           max_positions) -> None:
        head_range = None
        selected, kw, kb, vw, vb = [], [], [], [], []
        for name, t in zip(names, self.layers):
            required = {"selected", "k_weight", "k_bias", "v_weight", "v_bias"}
            missing = required.difference(t)
            if missing:
                raise ValueError(f"{name} is missing tensors: {sorted(missing)}")
            if "headwise" not in t:
                raise ValueError(f"{name} headwise=False does not match method=cachebridge")
            heads = int(t["k_bias"].shape[0])
            if heads % self.target_tp_size:
                raise ValueError(
                    f"target KV heads ({heads}) must divide target TP ({self.target_tp_size})")
            per = heads // self.target_tp_size
            rng = (self.target_tp_rank * per, self.target_tp_rank * per + per)
            if head_range is None:
                head_range = rng
            elif head_range != rng:
                raise ValueError("target-head geometry changes across mapper layers")
            cut = slice(*rng)
            sel = t["selected"].long().cpu()
            if sel.ndim != 1 or sel.numel() == 0:
                raise ValueError(f"{name}: selected must be a non-empty 1-D list")
            selected.append(sel)
            kw.append(t["k_weight"][cut].float())
            kb.append(t["k_bias"][cut].float())
            vw.append(t["v_weight"][cut].float())
            vb.append(t["v_bias"][cut].float())
        s = max(len(x) for x in selected)
        d = int(kb[0].shape[-1])
        lt, ht = len(self.layers), head_range[1] - head_range[0]
        al = torch.empty(lt, ht, s, dtype=torch.int64)
        ah = torch.empty(lt, ht, s, dtype=torch.int64)
        k_w = torch.zeros(lt, ht, s * d, d)
        v_w = torch.zeros(lt, ht, s * d, d)
        for l, sel in enumerate(selected):
            n = len(sel)
            if kw[l].shape != (ht, n * d, d) or vw[l].shape != (ht, n * d, d):
                raise ValueError("CacheBridge source-head geometry mismatch")
            # Shorter supports are padded with zero-weight repeats of their first source row.
            padded = torch.cat((sel, sel[:1].repeat(s - n)))
            al[l] = padded[None, :].expand(ht, s)
            ah[l] = torch.arange(head_range[0], head_range[1])[:, None].expand(ht, s)
            k_w[l, :, : n * d] = kw[l]
            v_w[l, :, : n * d] = vw[l]
        self._init_plan(assign_layer=al, assign_head=ah, k_weight=k_w, k_bias=torch.stack(kb),
                        v_weight=v_w, v_bias=torch.stack(vb), source_rope_theta=source_rope_theta,
                        target_rope_theta=target_rope_theta,
                        source_rope_scaling=source_rope_scaling,
                        target_rope_scaling=target_rope_scaling, dtype=dtype, device=device,
                        max_positions=max_positions, target_head_start=head_range[0],
                        target_head_stop=head_range[1])
