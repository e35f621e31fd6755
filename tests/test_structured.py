"""Structured-state installs (Gemma 3 roster, Qwen3.5 recurrent memory): host logic
and the oracle of the recurrent-state transform (CPU).

Reference tests restated (paths in the reference repository):
``tests/test_architectures.py:100-111`` (bilinear read-out of the transformed
state), ``:126-158`` (Gemma window and all-or-nothing install), ``:160-215``
(linear-state install), ``tests/test_architecture_caches.py:17-80`` (the same
installs into transformers' structured ``DynamicCache``).
"""

from __future__ import annotations

import ctypes
import inspect
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from cachebridge_amd import _lib, architectures as arch
from oracle import structured as osd


class AttentionLayer:
    def __init__(self, window=None):
        self.is_sliding = window is not None
        self.sliding_window = window
        self.is_initialized = False

    def update(self, key, value):
        self.keys, self.values = key, value
        self.is_initialized = True
        self.cumulative_length = key.shape[-2]


class RecurrentLayer:
    def __init__(self):
        self.has_previous_state = [False]
        self.recurrent_states, self.conv_states = {}, {}

    def update_conv_state(self, value, *, state_idx, conv_kernel_size):
        self.conv_states[state_idx] = value

    def update_recurrent_state(self, value, *, state_idx):
        self.recurrent_states[state_idx] = value
        self.has_previous_state[state_idx] = True


def _linear_spec(index=0):
    # linear_num_key_heads=1, linear_num_value_heads=2, key dim 3, value dim 5, kernel 4
    return arch.LinearLayerSpec(index=index, key_heads=1, value_heads=2, key_dim=3, value_dim=5,
                                conv_kernel_size=4)


# --- oracle of transform_delta_state --------------------------------------


def test_oracle_preserves_bilinear_readout_for_rectangular_bases():
    g = torch.Generator().manual_seed(7)
    source = torch.randn(2, 3, 4, generator=g, dtype=torch.float64)
    a = torch.randn(2, 3, 5, generator=g, dtype=torch.float64)
    b = torch.randn(2, 4, 6, generator=g, dtype=torch.float64)
    q = torch.randn(2, 1, 5, generator=g, dtype=torch.float64)
    mapped = torch.from_numpy(osd.transform_delta_state(source, a, b))
    expected = torch.einsum("hri,hji,hjk,hkl->hrl", q, a, source, b)
    torch.testing.assert_close(q @ mapped, expected)
    assert mapped.shape == (2, 5, 6)


def test_oracle_matches_explicit_sums_and_broadcasts():
    rng = np.random.default_rng(3)
    u, a, b = rng.standard_normal((3, 4)), rng.standard_normal((3, 2)), rng.standard_normal((4, 5))
    np.testing.assert_allclose(osd.transform_delta_state(u, a, b), osd.transform_delta_state_loops(u, a, b),
                               rtol=1e-13, atol=1e-13)
    ub = rng.standard_normal((6, 3, 4))
    out = osd.transform_delta_state(ub, a, b)  # bases shared by every batch entry
    for i in range(6):
        np.testing.assert_allclose(out[i], osd.transform_delta_state_loops(ub[i], a, b), rtol=1e-13, atol=1e-13)
    with pytest.raises(ValueError, match="do not match"):
        osd.transform_delta_state(u, rng.standard_normal((4, 2)), b)


def test_required_replay_is_kernel_minus_one():
    assert arch.required_replay(4) == 3
    with pytest.raises(ValueError, match="positive"):
        arch.required_replay(0)


def test_transform_rejects_bad_inputs_before_any_launch():
    u = torch.zeros(2, 3, 4)
    with pytest.raises(ValueError, match="matrix-valued"):
        arch.transform_delta_state(torch.zeros(3), torch.zeros(3, 2), torch.zeros(4, 2))
    with pytest.raises(ValueError, match="do not match"):
        arch.transform_delta_state(u, torch.zeros(2, 4, 5), torch.zeros(2, 4, 6))
    with pytest.raises(ValueError, match="one GPU"):  # no CPU path
        arch.transform_delta_state(u, torch.zeros(2, 3, 5), torch.zeros(2, 4, 6))


def test_delta_state_abi_validation_without_a_device():
    lib = _lib.load()
    call = lib.cb_delta_state_transform
    assert call(7, 1, 4, 4, 4, 4, None, 0, None, 0, None, 0, None, 0, None) == _lib.CB_EINVAL
    assert b"dtype" in lib.cb_last_error()
    assert call(_lib.CB_DTYPE_F32, 1, 0, 4, 4, 4, None, 0, None, 0, None, 0, None, 0, None) == _lib.CB_EINVAL
    assert call(_lib.CB_DTYPE_F32, 1, 4, 513, 4, 4, None, 0, None, 0, None, 0, None, 0, None) == _lib.CB_EINVAL
    assert b"512" in lib.cb_last_error()
    assert call(_lib.CB_DTYPE_F64, 2, 4, 4, 4, 4, None, 0, None, 0, None, 0, None, 0, None) == _lib.CB_EINVAL
    assert b"null" in lib.cb_last_error()
    assert call(_lib.CB_DTYPE_F64, 1, 4, 4, 4, 4, None, -1, None, 0, None, 0, None, 0, None) == _lib.CB_EINVAL
    # an empty batch is a no-op that touches nothing
    assert call(_lib.CB_DTYPE_F64, 0, 4, 4, 4, 4, None, 0, None, 0, None, 0, None, 0, None) == _lib.CB_OK


# --- Gemma 3 roster --------------------------------------------------------


def test_gemma_window_and_absolute_position_survive_installation():
    key = torch.arange(9 * 2 * 3).reshape(9, 2, 3).float()
    local = arch.materialize_kv(key, key + 1, layer_type="sliding_attention", sliding_window=4)
    full = arch.materialize_kv(key, key + 1, layer_type="full_attention", sliding_window=4)
    assert local.first_position == 6 and local.prefix_length == 9
    torch.testing.assert_close(local.key, key[-3:])
    cache = SimpleNamespace(layers=[AttentionLayer(4), AttentionLayer()])
    mapped = {i: (x.key.permute(1, 0, 2)[None], x.value.permute(1, 0, 2)[None])
              for i, x in enumerate((local, full))}
    arch.install_kv(cache, mapped=mapped, prefix_length=9)
    assert cache.layers[0].keys.shape[-2] == 3 and cache.layers[0].cumulative_length == 9
    assert cache.layers[1].keys.shape[-2] == 9


def test_invalid_later_gemma_payload_leaves_all_layers_unmodified():
    cache = SimpleNamespace(layers=[AttentionLayer(4), AttentionLayer()])
    local = torch.zeros(1, 2, 3, 8)
    invalid_full = torch.zeros(1, 2, 8, 8)
    with pytest.raises(ValueError, match="history length"):
        arch.install_kv(cache, mapped={0: (local, local), 1: (invalid_full, invalid_full)}, prefix_length=9)
    assert all(not layer.is_initialized for layer in cache.layers)
    with pytest.raises(ValueError, match="cover every"):
        arch.install_kv(cache, mapped={0: (local, local)}, prefix_length=9)
    with pytest.raises(ValueError, match="Unsupported"):
        arch.materialize_kv(torch.zeros(3, 1, 2), torch.zeros(3, 1, 2), layer_type="linear_attention",
                            sliding_window=4)


# --- Qwen3.5 linear / attention installs ------------------------------------


def test_recurrent_install_preserves_fp32_memory_and_bf16_convolution():
    spec = _linear_spec()
    cache = SimpleNamespace(layers=[RecurrentLayer()])
    recurrent = torch.randn(1, 2, 3, 5)
    conv = torch.randn(1, 16, 4, dtype=torch.bfloat16)
    assert spec.conv_channels == 16
    arch.install_linear_state(cache, 0, recurrent_state=recurrent, conv_state=conv, conv_kernel_size=4, spec=spec)
    assert cache.layers[0].has_previous_state[0]
    assert cache.layers[0].recurrent_states[0] is recurrent
    assert cache.layers[0].conv_states[0] is conv
    with pytest.raises(ValueError, match="previous state"):
        arch.install_linear_state(cache, 0, recurrent_state=recurrent, conv_state=conv, conv_kernel_size=4)


def test_recurrent_install_rejects_geometry_before_mutation():
    spec = _linear_spec()
    cache = SimpleNamespace(layers=[RecurrentLayer()])
    with pytest.raises(ValueError, match="Recurrent tensor"):
        arch.install_linear_state(cache, 0, recurrent_state=torch.zeros(1, 2, 4, 5),
                                  conv_state=torch.zeros(1, 16, 4), conv_kernel_size=4, spec=spec)
    with pytest.raises(ValueError, match="Convolution tensor"):
        arch.install_linear_state(cache, 0, recurrent_state=torch.zeros(1, 2, 3, 5),
                                  conv_state=torch.zeros(1, 15, 4), conv_kernel_size=4, spec=spec)
    with pytest.raises(ValueError, match="specification does not match"):
        arch.install_linear_state(cache, 0, recurrent_state=torch.zeros(1, 2, 3, 5),
                                  conv_state=torch.zeros(1, 16, 4), conv_kernel_size=4, spec=_linear_spec(1))
    with pytest.raises(ValueError, match="floating-point"):
        arch.install_linear_state(cache, 0, recurrent_state=torch.zeros(1, 2, 3, 5, dtype=torch.int32),
                                  conv_state=torch.zeros(1, 16, 4), conv_kernel_size=4)
    assert not cache.layers[0].conv_states and not cache.layers[0].recurrent_states


def test_attention_install_rejects_recurrent_destination():
    with pytest.raises(TypeError, match="full-attention"):
        arch.install_attention_kv(SimpleNamespace(layers=[RecurrentLayer()]), 0,
                                  torch.zeros(1, 1, 2, 4), torch.zeros(1, 1, 2, 4))
    with pytest.raises(TypeError, match="full-attention"):
        arch.install_attention_kv(SimpleNamespace(layers=[AttentionLayer(4)]), 0,
                                  torch.zeros(1, 1, 2, 4), torch.zeros(1, 1, 2, 4))
    layer = AttentionLayer()
    arch.install_attention_kv(SimpleNamespace(layers=[layer]), 0, torch.ones(1, 1, 2, 4), torch.ones(1, 1, 2, 4))
    with pytest.raises(ValueError, match="already initialized"):
        arch.install_attention_kv(SimpleNamespace(layers=[layer]), 0, torch.ones(1, 1, 2, 4),
                                  torch.ones(1, 1, 2, 4))


def _native_cache_type():
    transformers = pytest.importorskip("transformers")
    if "config" not in inspect.signature(transformers.DynamicCache).parameters:
        pytest.skip("Requires the config-driven structured DynamicCache interface")
    return transformers.DynamicCache


def test_native_gemma_cache_preserves_next_query_window_offset():
    cache_type = _native_cache_type()
    module = pytest.importorskip("transformers.models.gemma3.configuration_gemma3")
    cfg = module.Gemma3TextConfig(vocab_size=97, hidden_size=32, intermediate_size=64, num_hidden_layers=2,
                                  num_attention_heads=4, num_key_value_heads=2, head_dim=8, sliding_window=4,
                                  layer_types=["sliding_attention", "full_attention"])
    cache = cache_type(config=cfg)
    mapped = {}
    for index, kind in enumerate(cfg.layer_types):
        length = 3 if kind == "sliding_attention" else 9
        key = torch.randn(1, 2, length, 8)
        mapped[index] = key, torch.randn_like(key)
    arch.install_kv(cache, mapped=mapped, prefix_length=9)
    assert cache.layers[0].get_mask_sizes(1) == (4, 6)
    assert cache.layers[1].get_seq_length() == 9
    for index, layer in enumerate(cache.layers):
        torch.testing.assert_close(layer.keys, mapped[index][0])
        torch.testing.assert_close(layer.values, mapped[index][1])


def test_native_qwen35_cache_contains_all_continuation_states():
    cache_type = _native_cache_type()
    module = pytest.importorskip("transformers.models.qwen3_5.configuration_qwen3_5")
    cfg = module.Qwen3_5TextConfig(vocab_size=97, hidden_size=32, intermediate_size=64, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=8,
                                   linear_num_key_heads=1, linear_num_value_heads=2, linear_key_head_dim=4,
                                   linear_value_head_dim=4, linear_conv_kernel_dim=4,
                                   layer_types=["linear_attention", "full_attention"])
    cache = cache_type(config=cfg)
    spec = arch.LinearLayerSpec(index=0, key_heads=1, value_heads=2, key_dim=4, value_dim=4, conv_kernel_size=4)
    state = torch.randn(1, 2, 4, 4)
    conv = torch.randn(1, spec.conv_channels, 4, dtype=torch.bfloat16)
    arch.install_linear_state(cache, 0, recurrent_state=state, conv_state=conv, conv_kernel_size=4, spec=spec)
    key, value = torch.randn(1, 2, 9, 8), torch.randn(1, 2, 9, 8)
    arch.install_attention_kv(cache, 1, key, value)
    assert cache.layers[0].has_previous_state[0]
    torch.testing.assert_close(cache.layers[0].recurrent_states[0], state)
    torch.testing.assert_close(cache.layers[0].conv_states[0], conv)
