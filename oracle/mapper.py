"""Oracle restatement of the reference ``PageMapper`` (``cb/mapper.py:17-239``).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

``map_page`` follows ``cb/mapper.py:117-239`` op for op in torch fp32:
un-rotate all source keys with the source RoPE, build the per-target-layer
feature tensor by concatenating the ``selected`` source layers in list order,
slice the target heads, contract with the fp32 head-wise weights plus bias,
rotate the stacked keys with the target RoPE and cast to the source dtype.

Parity pinned by: golden outputs written from the reference
(``tests/golden/*.safetensors``: the toy fp32 configuration in full, and a
D=128 bf16 slice with s=1 and s=8 supports), the closed-form affine fixtures of
the reference tests (``tests/test_fitting.py:48-90``,
``examples/fit_and_map.py:20-46``: target = a*src_i + b*src_j + c with exact
weights), identity maps (``tests/test_mapper.py:53-105``) and an fp64
brute-force contraction on tiny inputs.
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import torch
from torch import Tensor

from .rope import apply_rope, qwen_rope, remove_rope


@dataclass(frozen=True)
class LayerWeights:
    """``cb/mapper.py:17-24``."""

    selected: Tensor
    k_weight: Tensor
    k_bias: Tensor
    v_weight: Tensor
    v_bias: Tensor
    headwise: bool


class PageMapper:
    """``cb/mapper.py:27-239`` (full-input mapper; head-wise and dense maps)."""

    def __init__(
        self,
        mapper_dir,
        *,
        method: str,
        source_rope_theta: float,
        target_rope_theta: float,
        source_rope_scaling: dict | None = None,
        target_rope_scaling: dict | None = None,
        device="cpu",
        target_tp_rank: int = 0,
        target_tp_size: int = 1,
        _tensors: list[dict] | None = None,
    ) -> None:
        from safetensors.torch import load_file

        self.method = method
        self.source_rope_theta = float(source_rope_theta)
        self.target_rope_theta = float(target_rope_theta)
        self.source_rope_scaling = source_rope_scaling
        self.target_rope_scaling = target_rope_scaling
        self.device = torch.device(device)
        self.target_tp_rank = int(target_tp_rank)
        self.target_tp_size = int(target_tp_size)
        self.target_head_start: int | None = None
        self.target_head_stop: int | None = None
        if _tensors is None:
            paths = sorted(Path(mapper_dir).glob("layer_*.safetensors"))
            if not paths:
                raise FileNotFoundError(f"no layer_*.safetensors in {mapper_dir}")
            sources = [(str(p), load_file(p, device=str(self.device))) for p in paths]
        else:
            sources = [(f"layer {i}", t) for i, t in enumerate(_tensors)]
        self.layers: list[LayerWeights] = []
        for name, tensors in sources:
            self.layers.append(self._slice_layer(name, tensors))

    @classmethod
    def from_tensors(cls, layers: list[dict], **kwargs) -> "PageMapper":
        """Build from in-memory ``layer_*.safetensors`` dictionaries."""
        return cls(None, _tensors=layers, **kwargs)

    def _slice_layer(self, name: str, tensors: dict) -> LayerWeights:
        """``cb/mapper.py:64-110``: schema check and TP head slice."""
        required = {"selected", "k_weight", "k_bias", "v_weight", "v_bias"}
        missing = required.difference(tensors)
        if missing:
            raise ValueError(f"{name} is missing tensors: {sorted(missing)}")
        headwise = "headwise" in tensors
        if headwise != (self.method == "cachebridge"):
            raise ValueError(f"{name} headwise={headwise} does not match method={self.method}")
        heads = int(tensors["k_bias"].shape[0])
        if heads % self.target_tp_size:
            raise ValueError(
                f"target KV heads ({heads}) must divide target TP ({self.target_tp_size})"
            )
        per_rank = heads // self.target_tp_size
        start = self.target_tp_rank * per_rank
        stop = start + per_rank
        if self.target_head_start is None:
            self.target_head_start, self.target_head_stop = start, stop
        elif (self.target_head_start, self.target_head_stop) != (start, stop):
            raise ValueError("target-head geometry changes across mapper layers")
        cut = slice(start, stop)

        def weight(key: str) -> Tensor:
            w = tensors[key]
            return (w[cut] if headwise else w[:, cut]).contiguous()

        return LayerWeights(
            selected=tensors["selected"].long().cpu(),
            k_weight=weight("k_weight"),
            k_bias=tensors["k_bias"][cut].contiguous(),
            v_weight=weight("v_weight"),
            v_bias=tensors["v_bias"][cut].contiguous(),
            headwise=headwise,
        )

    @property
    def target_layers(self) -> int:
        return len(self.layers)

    @torch.inference_mode()
    def map_page(
        self,
        source_page: Tensor,
        *,
        position_start: int,
        source_head_offset: int = 0,
        output_device="cpu",
        output: Tensor | None = None,
    ) -> Tensor:
        """``cb/mapper.py:117-239``."""
        if source_page.ndim != 5 or source_page.shape[0] != 2:
            raise ValueError("source page must be [2,layers,tokens,kv_heads,head_dim]")
        page = source_page.to(self.device)
        dtype = page.dtype
        _, depth, tokens, _, dim = page.shape
        positions = torch.arange(
            position_start, position_start + tokens, device=self.device, dtype=torch.long
        )
        cos_s, sin_s = qwen_rope(
            positions, head_dim=dim, theta=self.source_rope_theta,
            scaling=self.source_rope_scaling,
        )
        keys = remove_rope(page[0].float(), cos_s, sin_s)
        values = page[1].float()
        lo = self.target_head_start - source_head_offset
        hi = self.target_head_stop - source_head_offset
        out_k: list[Tensor] = []
        out_v: list[Tensor] = []
        for layer in self.layers:
            chosen = layer.selected.tolist()
            if not chosen or max(chosen) >= depth:
                raise ValueError("mapper selected layer exceeds source page depth")
            if layer.headwise:
                fk = torch.cat([keys[i] for i in chosen], dim=-1)[:, lo:hi]
                fv = torch.cat([values[i] for i in chosen], dim=-1)[:, lo:hi]
                if fk.shape[1] != layer.k_weight.shape[0]:
                    raise ValueError("CacheBridge source-head geometry mismatch")
                yk = torch.einsum("thf,hfd->thd", fk, layer.k_weight.float()) + layer.k_bias.float()
                yv = torch.einsum("thf,hfd->thd", fv, layer.v_weight.float()) + layer.v_bias.float()
            else:
                fk = torch.cat([keys[i].reshape(tokens, -1) for i in chosen], dim=-1)
                fv = torch.cat([values[i].reshape(tokens, -1) for i in chosen], dim=-1)
                if fk.shape[-1] != layer.k_weight.shape[0]:
                    raise ValueError("NV Dense feature-width mismatch")
                heads, width = layer.k_bias.shape
                yk = (
                    fk @ layer.k_weight.float().reshape(fk.shape[-1], -1)
                    + layer.k_bias.float().reshape(-1)
                ).reshape(tokens, heads, width)
                yv = (
                    fv @ layer.v_weight.float().reshape(fv.shape[-1], -1)
                    + layer.v_bias.float().reshape(-1)
                ).reshape(tokens, heads, width)
            out_k.append(yk)
            out_v.append(yv)
        tk = torch.stack(out_k, dim=0)
        tv = torch.stack(out_v, dim=0)
        cos_t, sin_t = qwen_rope(
            positions, head_dim=tk.shape[-1], theta=self.target_rope_theta,
            scaling=self.target_rope_scaling,
        )
        tk = apply_rope(tk, cos_t, sin_t)
        if output is None:
            return torch.stack((tk, tv), dim=0).to(device=output_device, dtype=dtype)
        expected = (2, self.target_layers, tokens, tk.shape[2], tk.shape[3])
        if (
            tuple(output.shape) != expected
            or output.dtype != dtype
            or output.device != torch.device(output_device)
        ):
            raise ValueError("preallocated mapper output geometry/dtype/device mismatch")
        output[0].copy_(tk)
        output[1].copy_(tv)
        return output


class HeadLocalPageMapper(PageMapper):
    """``cb/online/mapping.py:6-33``: slice the needed heads before mapping."""

    def map_page(self, source_page, *, position_start, source_head_offset=0,
                 output_device="cpu", output=None):
        if self.method == "cachebridge":
            start = self.target_head_start - source_head_offset
            stop = self.target_head_stop - source_head_offset
            if not 0 <= start < stop <= source_page.shape[3]:
                raise ValueError("Received source shard does not contain required heads")
            source_page = source_page[:, :, :, start:stop, :]
            source_head_offset = self.target_head_start
        return super().map_page(
            source_page, position_start=position_start,
            source_head_offset=source_head_offset,
            output_device=output_device, output=output,
        )


def brute_force_map(
    source_page: Tensor,
    layers: list[dict],
    *,
    position_start: int,
    source_theta: float,
    target_theta: float,
) -> Tensor:
    """fp64 brute force of the head-wise map on tiny inputs (no reference code path).

    Un-rotates each key pair in fp64 with the exact angle, contracts in fp64,
    rotates with the target angle. Used to check the oracle's fp32 restatement
    within fp32 rounding error, independent of torch's fp32 kernels.
    """
    page = source_page.double()
    _, _, tokens, heads, dim = page.shape
    half = dim // 2
    j = torch.arange(half, dtype=torch.float64)
    pos = torch.arange(position_start, position_start + tokens, dtype=torch.float64)

    def angles(theta):
        inv = 1.0 / (theta ** (2 * j / dim))
        a = pos[:, None] * inv[None, :]
        return torch.cos(a)[None, :, None, :], torch.sin(a)[None, :, None, :]

    c, s = angles(source_theta)
    k1, k2 = page[0][..., :half], page[0][..., half:]
    # inverse rotation by angle a: (k1 c + k2 s, k2 c - k1 s)
    keys = torch.cat((k1 * c + k2 * s, k2 * c - k1 * s), dim=-1)
    values = page[1]
    out_k, out_v = [], []
    for layer in layers:
        chosen = [int(x) for x in layer["selected"].tolist()]
        fk = torch.cat([keys[i] for i in chosen], dim=-1)
        fv = torch.cat([values[i] for i in chosen], dim=-1)
        wk, wv = layer["k_weight"].double(), layer["v_weight"].double()
        out_k.append(torch.einsum("thf,hfd->thd", fk, wk) + layer["k_bias"].double())
        out_v.append(torch.einsum("thf,hfd->thd", fv, wv) + layer["v_bias"].double())
    tk = torch.stack(out_k)
    c, s = angles(target_theta)
    y1, y2 = tk[..., :half], tk[..., half:]
    tk = torch.cat((y1 * c - y2 * s, y2 * c + y1 * s), dim=-1)
    return torch.stack((tk, torch.stack(out_v)))
