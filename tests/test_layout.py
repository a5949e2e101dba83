"""KVCacheLayout: shapes and strides against torch's own strides of a tensor
of that shape (the reference formulas, flexkv/common/storage.py:59-149)."""
import pytest
import torch

from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType as T


def _torch_strides(layout):
    st = torch.empty(layout.kv_shape, dtype=torch.int8, device="meta").stride()
    if layout.type == T.LAYERWISE:
        return {"layer": st[0], "kv": st[1], "block": st[2]}
    return {"block": st[0], "layer": st[1], "kv": st[2]}


@pytest.mark.parametrize("kind", [T.LAYERWISE, T.BLOCKWISE])
@pytest.mark.parametrize("mla", [False, True])
@pytest.mark.parametrize("dims", [(32, 4096, 16, 8, 128), (80, 8192, 16, 1, 128),
                                  (61, 4096, 64, 1, 576), (3, 5, 2, 7, 11)])
def test_strides_match_torch(kind, mla, dims):
    L, N, t, h, d = dims
    lay = KVCacheLayout(kind, L, N, t, h, d, is_mla=mla)
    kv = 1 if mla else 2
    if kind == T.LAYERWISE:
        assert tuple(lay.kv_shape) == (L, kv, N, t, h, d)
    else:
        assert tuple(lay.kv_shape) == (N, L, kv, t, h, d)
    ref = _torch_strides(lay)
    assert lay.get_layer_stride() == ref["layer"]
    assert lay.get_kv_stride() == ref["kv"]
    assert lay.get_block_stride() == ref["block"]
    assert lay.get_chunk_size() == t * h * d
    assert lay.get_total_elements() == L * kv * N * t * h * d
    assert lay.get_elements_per_block() == L * kv * t * h * d


def test_div_and_equality():
    lay = KVCacheLayout(T.LAYERWISE, 32, 4096, 16, 8, 128)
    per = lay.div_layer(32)
    assert per.num_layer == 1 and per.get_kv_stride() == 4096 * 16 * 8 * 128
    assert per.get_block_stride() == 16 * 8 * 128
    assert lay.div_head(8).num_head == 1
    assert lay.div_block(3, padding=True).num_block == 1366
    with pytest.raises(AssertionError):
        lay.div_block(3)
    with pytest.raises(AssertionError):
        lay.div_layer(5)
    assert lay == KVCacheLayout(T.LAYERWISE, 32, 4096, 16, 8, 128)
    assert lay != KVCacheLayout(T.BLOCKWISE, 32, 4096, 16, 8, 128)


def test_byte_strides():
    lay = KVCacheLayout(T.BLOCKWISE, 32, 16384, 16, 8, 128)
    chunk, kv, layer, block = lay.byte_strides(torch.bfloat16)
    assert chunk == 32768 and kv == 32768 and layer == 65536 and block == 2 << 20


def test_invalid_type():
    with pytest.raises(ValueError):
        KVCacheLayout("ROWWISE", 1, 1, 1, 1, 1)
