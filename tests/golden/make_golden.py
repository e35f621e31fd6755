"""Write golden vectors for the handoff path from the reference implementation.

Run in the development container only (the reference tree is not present on
GPU machines):

    PYTHONPATH=/root/reference/src python tests/golden/make_golden.py

It imports ``cachebridge.rope`` and ``cachebridge.mapper`` from the reference
(read-only) and records, for seeded synthetic inputs, the reference outputs of
exactly the functions that no closed form pins bit for bit:

- ``rope_tables.safetensors``: ``qwen_rope`` at positions {0, 1, 4095, 32767,
  40959} for theta {1e4, 1e6}, head_dim {64, 128}, plus a YaRN scaling dict.
- ``toy_fp32.safetensors``: the toy fp32 configuration in full (source 8x2,
  target 12x2, head_dim 64, 256 tokens, per-(layer, head) random source
  assignment), mapped by the reference ``PageMapper`` over the virtual page.
- ``slice_bf16_s1.safetensors``: D=128 bf16 slice, 4 target layers x 2 heads,
  64 tokens at positions 4032-4095, s=1 random assignment, theta 1e6.
- ``slice_bf16_s8.safetensors``: D=128 bf16, head-identity reference artifact
  with an unsorted s=8 support list, TP 2 rank 1, 32 tokens at 1000-1031,
  theta 1e4 -> 1e6.
- ``slice_bf16_yarn.safetensors``: D=128 bf16, s=1, YaRN on both sides,
  positions 40000-40031.

Inputs are stored next to outputs (torch RNG streams may change between
versions); seeds are recorded in ``manifest.json``.
"""

from __future__ import annotations

import json
import math
import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

REFERENCE_SRC = "/root/reference/src"
OUT = Path(__file__).resolve().parent

YARN = {"rope_type": "yarn", "factor": 4.0, "original_max_position_embeddings": 32768}


def reference():
    if REFERENCE_SRC not in sys.path:
        sys.path.insert(0, REFERENCE_SRC)
    from cachebridge import mapper, rope  # noqa: E402

    return mapper, rope


def virtual_page(page, assign_layer, assign_head):
    lt, ht, s = assign_layer.shape
    out = page.new_empty(2, lt * s, page.shape[2], ht, page.shape[4])
    for l in range(lt):
        for h in range(ht):
            for k in range(s):
                out[:, l * s + k, :, h] = page[:, int(assign_layer[l, h, k]), :, int(assign_head[l, h, k])]
    return out


def layer_files(spec):
    lt, _, s = spec["assign_layer"].shape
    files = []
    for l in range(lt):
        files.append({
            "selected": torch.tensor([l * s + k for k in range(s)], dtype=torch.int64),
            "k_weight": spec["k_weight"][l].contiguous(),
            "k_bias": spec["k_bias"][l].contiguous(),
            "v_weight": spec["v_weight"][l].contiguous(),
            "v_bias": spec["v_bias"][l].contiguous(),
            "headwise": torch.tensor(1, dtype=torch.int8),
        })
    return files


def run_mapper(mapper_mod, files, tmp, **kwargs):
    tmp.mkdir(parents=True, exist_ok=True)
    for old in tmp.glob("layer_*.safetensors"):
        old.unlink()
    for i, tensors in enumerate(files):
        save_file(tensors, str(tmp / f"layer_{i:03d}.safetensors"))
    return mapper_mod.PageMapper(tmp, method="cachebridge", **kwargs)


def random_assignment(gen, lt, ht, hs, selected, s=1):
    pick = torch.randint(0, len(selected), (lt, ht, s), generator=gen)
    layer = torch.tensor(selected, dtype=torch.int64)[pick]
    head = torch.randint(0, hs, (lt, ht, s), generator=gen)
    return layer, head


def maps(gen, lt, ht, s, d):
    shape_w = (lt, ht, s * d, d)
    return {
        "k_weight": torch.randn(shape_w, generator=gen) / math.sqrt(s * d),
        "v_weight": torch.randn(shape_w, generator=gen) / math.sqrt(s * d),
        "k_bias": torch.randn(lt, ht, d, generator=gen) * 0.1,
        "v_bias": torch.randn(lt, ht, d, generator=gen) * 0.1,
    }


def main():
    mapper_mod, rope_mod = reference()
    manifest = {"reference": "WHU-XingyuQu/CacheBridge src/cachebridge (rope.py, mapper.py)",
                "torch": torch.__version__, "files": {}}
    tmp = OUT / "_tmp_mapper"
    torch.set_num_threads(1)

    # 1. RoPE tables.
    positions = torch.tensor([0, 1, 4095, 32767, 40959])
    tables = {"positions": positions}
    for d in (64, 128):
        for theta in (1e4, 1e6):
            c, s_ = rope_mod.qwen_rope(positions, head_dim=d, theta=theta)
            tables[f"cos_d{d}_t{int(theta)}"], tables[f"sin_d{d}_t{int(theta)}"] = c, s_
        c, s_ = rope_mod.qwen_rope(positions, head_dim=d, theta=1e6, scaling=YARN)
        tables[f"cos_d{d}_yarn"], tables[f"sin_d{d}_yarn"] = c, s_
    save_file(tables, str(OUT / "rope_tables.safetensors"))
    manifest["files"]["rope_tables.safetensors"] = {"yarn": YARN}

    # 2. Toy fp32 configuration (source 8x2 -> target 12x2, D 64, 256 tokens).
    gen = torch.Generator().manual_seed(1001)
    d, ls, hs, lt, ht, n = 64, 8, 2, 12, 2, 256
    page = torch.randn(2, ls, n, hs, d, generator=gen)
    selected = sorted(torch.randperm(ls, generator=gen)[:4].tolist())
    al, ah = random_assignment(gen, lt, ht, hs, selected)
    spec = {"assign_layer": al, "assign_head": ah, **maps(gen, lt, ht, 1, d)}
    m = run_mapper(mapper_mod, layer_files(spec), tmp, source_rope_theta=1e4, target_rope_theta=1e6)
    out = m.map_page(virtual_page(page, al, ah), position_start=0)
    save_file({"page": page, "out": out, **spec}, str(OUT / "toy_fp32.safetensors"))
    manifest["files"]["toy_fp32.safetensors"] = {
        "seed": 1001, "selected": selected, "position_start": 0,
        "source_theta": 1e4, "target_theta": 1e6, "dtype": "float32"}

    # 3. D=128 bf16 slice, s=1, positions 4032-4095.
    gen = torch.Generator().manual_seed(2002)
    d, ls, hs, lt, ht, n = 128, 8, 2, 4, 2, 64
    scale = torch.exp(torch.randn(d, generator=gen) * 0.5)
    page = (torch.randn(2, ls, n, hs, d, generator=gen) * scale).to(torch.bfloat16)
    selected = [0, 2, 5, 7]
    al, ah = random_assignment(gen, lt, ht, hs, selected)
    spec = {"assign_layer": al, "assign_head": ah, **maps(gen, lt, ht, 1, d)}
    m = run_mapper(mapper_mod, layer_files(spec), tmp, source_rope_theta=1e6, target_rope_theta=1e6)
    out = m.map_page(virtual_page(page, al, ah), position_start=4032)
    save_file({"page": page, "out": out, **spec}, str(OUT / "slice_bf16_s1.safetensors"))
    manifest["files"]["slice_bf16_s1.safetensors"] = {
        "seed": 2002, "position_start": 4032, "source_theta": 1e6, "target_theta": 1e6,
        "dtype": "bfloat16"}

    # 4. D=128 bf16, reference-format head-identity artifact, s=8 unsorted support, TP 2 rank 1.
    gen = torch.Generator().manual_seed(3003)
    d, ls, hs, n = 128, 12, 2, 32
    support = [3, 1, 0, 9, 11, 4, 6, 8]
    page = (torch.randn(2, ls, n, hs, d, generator=gen) * scale).to(torch.bfloat16)
    w = maps(gen, 1, 2, len(support), d)
    files = [{"selected": torch.tensor(support, dtype=torch.int64),
              "k_weight": w["k_weight"][0].contiguous(), "k_bias": w["k_bias"][0].contiguous(),
              "v_weight": w["v_weight"][0].contiguous(), "v_bias": w["v_bias"][0].contiguous(),
              "headwise": torch.tensor(1, dtype=torch.int8)}]
    m = run_mapper(mapper_mod, files, tmp, source_rope_theta=1e4, target_rope_theta=1e6,
                   target_tp_rank=1, target_tp_size=2)
    out = m.map_page(page, position_start=1000)
    compact = m.map_page(page[:, :, :, 1:2], position_start=1000, source_head_offset=1)
    assert torch.equal(out, compact)
    save_file({"page": page, "out": out, **{k: v[0].contiguous() for k, v in w.items()},
               "selected": files[0]["selected"]}, str(OUT / "slice_bf16_s8.safetensors"))
    manifest["files"]["slice_bf16_s8.safetensors"] = {
        "seed": 3003, "support": support, "position_start": 1000, "source_theta": 1e4,
        "target_theta": 1e6, "target_tp_rank": 1, "target_tp_size": 2, "dtype": "bfloat16"}

    # 5. YaRN on both sides, positions beyond the original window.
    gen = torch.Generator().manual_seed(4004)
    d, ls, hs, lt, ht, n = 128, 4, 2, 2, 2, 32
    page = (torch.randn(2, ls, n, hs, d, generator=gen) * scale).to(torch.bfloat16)
    al, ah = random_assignment(gen, lt, ht, hs, [1, 3])
    spec = {"assign_layer": al, "assign_head": ah, **maps(gen, lt, ht, 1, d)}
    m = run_mapper(mapper_mod, layer_files(spec), tmp, source_rope_theta=1e6, target_rope_theta=1e6,
                   source_rope_scaling=YARN, target_rope_scaling=YARN)
    out = m.map_page(virtual_page(page, al, ah), position_start=40000)
    save_file({"page": page, "out": out, **spec}, str(OUT / "slice_bf16_yarn.safetensors"))
    manifest["files"]["slice_bf16_yarn.safetensors"] = {
        "seed": 4004, "position_start": 40000, "source_theta": 1e6, "target_theta": 1e6,
        "yarn": YARN, "dtype": "bfloat16"}

    for old in tmp.glob("layer_*.safetensors"):
        old.unlink()
    tmp.rmdir()
    (OUT / "manifest.json").write_text(json.dumps(manifest, indent=1) + "\n")
    print("wrote", sorted(manifest["files"]))


if __name__ == "__main__":
    main()
