"""torch.ops.dartkv.*: the HIP entry points registered as PyTorch operators (dartkv_amd/torch_ops.py).

CPU: the fake implementations give the shapes and dtypes of the real outputs on meta tensors, and the
decode operator rejects an unknown cache handle.  GPU: every operator returns the bytes of the Python
API it wraps, passes torch.library.opcheck (schema, fake tensors, AOT dispatch), and traces whole under
torch.compile.
"""

from __future__ import annotations

import pytest
import torch

from tests.golden_util import bits_equal

DEV = "cuda"


def _ops():
    import dartkv_amd  # noqa: F401  (registers the operators)
    return torch.ops.dartkv


@pytest.mark.parametrize("n,bits,group", [(100, 2, 64), (128, 4, 32), (7, 8, 64), (300, 2, 128)])
def test_fake_row_shapes(n, bits, group):
    ops = _ops()
    x = torch.empty(3, 5, n, device="meta", dtype=torch.bfloat16)
    values, scale, zero = ops.quantize_rows(x, bits, group, torch.float16)
    groups = -(-n // group)
    assert values.shape == (3, 5, -(-groups * group * bits // 8)) and values.dtype == torch.uint8
    assert scale.shape == zero.shape == (3, 5, groups) and scale.dtype == torch.float16
    assert ops.quantize_rows(x, bits, group, None)[1].dtype == torch.bfloat16  # metadata follows the data
    out = ops.dequantize_rows(values, scale, zero, bits, group, n, torch.float32)
    assert out.shape == (3, 5, n) and out.dtype == torch.float32


@pytest.mark.parametrize("T,group,ratio", [(130, 128, 0.25), (64, 32, 0.0), (16, 16, 1.0)])
def test_fake_mixed_key_shapes(T, group, ratio):
    ops = _ops()
    k = torch.empty(2, 4, T, 128, device="meta", dtype=torch.bfloat16)
    low, high, idx, scale, zero = ops.quantize_key_mixed(k, group, ratio, "magnitude", None, None)
    G, K, nb = -(-T // group), int(128 * ratio + 1e-6), (group + 3) // 4
    assert low.shape == (2, 4, 128, G, nb) and high.shape == (2, 4, K, G, nb if K else 4 * nb)
    assert idx.shape == (2, 4, K) and idx.dtype == torch.int32
    assert scale.shape == zero.shape == (2, 4, 128, G) and scale.dtype == torch.bfloat16
    assert ops.dequantize_key_mixed(low, high, idx, scale, zero, T, group, torch.float16).shape == (2, 4, T, 128)


def test_decode_operator_needs_a_registered_cache():
    ops = _ops()
    q = torch.empty(1, 4, 1, 128, device="meta", dtype=torch.bfloat16)
    assert ops.decode_attention(q, 1, None).shape == (1, 4, 1, 128)
    with pytest.raises(ValueError, match="unknown DartKVCache handle"):
        ops.decode_attention(torch.zeros(1, 4, 1, 128), 1, None)


@pytest.mark.gpu
def test_operators_return_the_python_api_bytes_and_pass_opcheck():
    import dartkv_amd as dart
    from dartkv_amd import synthetic
    from dartkv_amd.torch_ops import cache_handle
    ops = _ops()
    torch.manual_seed(2)
    x = torch.randn(6, 3, 200, device=DEV, dtype=torch.bfloat16)
    ref = dart.quantize(x, bits=4, group_size=64, metadata_dtype=torch.float16)
    values, scale, zero = ops.quantize_rows(x, 4, 64, torch.float16)
    assert bits_equal(values, ref.values) and bits_equal(scale, ref.scale) and bits_equal(zero, ref.zero_point)
    assert bits_equal(ops.dequantize_rows(values, scale, zero, 4, 64, 200, torch.bfloat16),
                      ref.dequantize(dtype=torch.bfloat16))
    k, v, q = synthetic.outlier_kv(2, 4, 300, 128, query_heads=16, dtype=torch.bfloat16, seed=4, device=DEV)
    mk = dart.quantize_key_mixed(k, group_size=128, promote_ratio=0.25, strategy="variance")
    fields = ops.quantize_key_mixed(k, 128, 0.25, "variance", None, None)
    for a, b in zip(fields, (mk.low_values, mk.high_values, mk.channel_indices, mk.scale, mk.zero_point)):
        assert bits_equal(a, b)
    assert bits_equal(ops.dequantize_key_mixed(*fields, 300, 128, torch.bfloat16), mk.dequantize(dtype=torch.bfloat16))
    cache = dart.DartKVCache(dart.DartKVCacheConfig(bits=2, page_size=128, key_group_size=128, value_group_size=64,
                                                    promote_ratio=0.25, sink_tokens=32, hold_partial_pages=True,
                                                    metadata_dtype=torch.float16))
    cache.append(k, v)
    handle = cache_handle(cache)
    assert bits_equal(ops.decode_attention(q, handle, None), dart.decode_attention(q, cache))
    for op, args in ((ops.quantize_rows.default, (x, 4, 64, torch.float16)),
                     (ops.dequantize_rows.default, (values, scale, zero, 4, 64, 200, torch.bfloat16)),
                     (ops.quantize_key_mixed.default, (k, 128, 0.25, "magnitude", None, None)),
                     (ops.dequantize_key_mixed.default, (*fields, 300, 128, torch.bfloat16)),
                     (ops.decode_attention.default, (q, handle, None))):
        torch.library.opcheck(op, args)


@pytest.mark.gpu
def test_operators_trace_whole_under_torch_compile():
    """A function of the operators compiles with fullgraph=True (no graph break into ctypes) and gives the
    eager bytes."""
    ops = _ops()
    torch.manual_seed(3)
    x = torch.randn(8, 256, device=DEV, dtype=torch.float16)

    def roundtrip(t):
        values, scale, zero = ops.quantize_rows(t, 2, 64, None)
        return ops.dequantize_rows(values, scale, zero, 2, 64, t.shape[-1], t.dtype)

    compiled = torch.compile(roundtrip, backend="aot_eager", fullgraph=True)
    assert bits_equal(compiled(x), roundtrip(x))
