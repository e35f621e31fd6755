"""GPU: the recurrent-state transform ``A^T U B`` against the float64 oracle.

``transform_delta_state`` (``cb/architectures/qwen35.py:52-61``) runs as one
launch of ``cb_delta_state_transform`` (16x16x4 MFMAs in the inputs' dtype).
Tolerances: float64 inputs agree with the oracle to 1e-12 relative to the
result's scale; float32 inputs to 2e-6 (fp32 products accumulated over k + v
terms). The reference's bilinear read-out test is restated on the GPU result.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cachebridge_amd import architectures as arch
from oracle import structured as osd

pytestmark = pytest.mark.gpu

RTOL = {torch.float64: 1e-12, torch.float32: 2e-6}


def _check(out, u, a, b):
    ref = osd.transform_delta_state(u.cpu(), a.cpu(), b.cpu())
    got = out.cpu().double().numpy()
    assert got.shape == ref.shape
    scale = np.abs(ref).max() + 1e-300
    err = np.abs(got - ref).max() / scale
    assert err <= RTOL[out.dtype], (err, out.dtype)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("lead,k,v,kp,vp", [
    ((2,), 3, 4, 5, 6),        # the reference's rectangular bases
    ((1,), 4, 4, 4, 4),
    ((3,), 128, 128, 128, 128),  # Qwen3.5 DeltaNet head (key/value dim 128)
    ((5,), 17, 33, 20, 7),     # no dimension a multiple of 16
    ((2,), 64, 512, 48, 96),   # the largest value dimension
    ((2, 3), 32, 16, 16, 40),  # two batch dimensions
])
def test_transform_matches_oracle(dtype, lead, k, v, kp, vp):
    print(f"delta state {dtype} lead={lead} k={k} v={v} kp={kp} vp={vp}", flush=True)
    g = torch.Generator().manual_seed(k * 1000 + v)
    u = torch.randn(*lead, k, v, generator=g, dtype=dtype)
    a = torch.randn(*lead, k, kp, generator=g, dtype=dtype)
    b = torch.randn(*lead, v, vp, generator=g, dtype=dtype)
    out = arch.transform_delta_state(u.cuda(), a.cuda(), b.cuda())
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == (*lead, kp, vp)
    _check(out, u, a, b)


@pytest.mark.parametrize("shared_key_basis", [False, True])
def test_many_entries_on_the_square_path(shared_key_basis):
    # The 128 x 128 fp32 path at a Qwen3.5-like batch (more entries than
    # resident workgroups, so several dispatch waves), with the key basis per
    # entry and shared by every entry (batch stride 0).
    g = torch.Generator().manual_seed(23)
    u = torch.randn(1300, 128, 128, generator=g)
    a = torch.randn(128, 128, generator=g) if shared_key_basis else torch.randn(1300, 128, 128, generator=g)
    b = torch.randn(1300, 128, 128, generator=g)
    out = arch.transform_delta_state(u.cuda(), a.cuda(), b.cuda())
    torch.cuda.synchronize()
    assert out.shape == (1300, 128, 128)
    _check(out, u, a, b)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_shared_bases_broadcast_over_the_batch(dtype):
    g = torch.Generator().manual_seed(11)
    u = torch.randn(4, 6, 24, 40, generator=g, dtype=dtype)   # [batch, heads, k, v]
    a = torch.randn(6, 24, 18, generator=g, dtype=dtype)      # per-head key basis
    b = torch.randn(40, 36, generator=g, dtype=dtype)         # one value basis
    out = arch.transform_delta_state(u.cuda(), a.cuda(), b.cuda())
    torch.cuda.synchronize()
    assert out.shape == (4, 6, 18, 36)
    _check(out, u, a, b)


def test_bilinear_readout_on_the_gpu_result():
    g = torch.Generator().manual_seed(7)
    source = torch.randn(2, 3, 4, generator=g, dtype=torch.float64)
    a = torch.randn(2, 3, 5, generator=g, dtype=torch.float64)
    b = torch.randn(2, 4, 6, generator=g, dtype=torch.float64)
    q = torch.randn(2, 1, 5, generator=g, dtype=torch.float64)
    mapped = arch.transform_delta_state(source.cuda(), a.cuda(), b.cuda()).cpu()
    expected = torch.einsum("hri,hji,hjk,hkl->hrl", q, a, source, b)
    torch.testing.assert_close(q @ mapped, expected)
    assert mapped.shape == (2, 5, 6)


def test_empty_batch_and_limits():
    out = arch.transform_delta_state(torch.zeros(0, 4, 4, device="cuda"), torch.zeros(4, 3, device="cuda"),
                                     torch.zeros(4, 2, device="cuda"))
    assert out.shape == (0, 3, 2)
    with pytest.raises(ValueError, match="512"):
        arch.transform_delta_state(torch.zeros(1, 4, 513, device="cuda"), torch.zeros(4, 3, device="cuda"),
                                   torch.zeros(513, 2, device="cuda"))
    with pytest.raises(ValueError, match="dtype"):
        arch.transform_delta_state(torch.zeros(1, 4, 4, device="cuda"), torch.zeros(4, 3, device="cuda"),
                                   torch.zeros(4, 2, device="cuda", dtype=torch.float64))
