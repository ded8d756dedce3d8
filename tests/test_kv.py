"""Host logic of the KV cache layout: block manager (test/kv/block_manager.jl), INT8
pool pairing (src/ops/quant.jl:104-135), rotary tables (src/model/rope.jl). CPU only."""
import math

import numpy as np
import pytest
import torch

import tileinfer_hip as ti


def test_block_manager():
    # test/kv/block_manager.jl:1-29
    b = ti.BlockManager(6, 4)
    s = ti.Sequence()
    ti.reserve(b, s, 5)
    assert s.block_table == [1, 2] and b.num_free_pages() == 4
    s.tokens.extend(range(1, 6))
    ti.reserve(b, s, 3)
    assert s.block_table == [1, 2]
    ti.reserve(b, s, 4)
    assert s.block_table == [1, 2, 3]
    other = ti.Sequence()
    ti.reserve(b, other, 1)
    assert ti.slots(b, s, 3, 3) == [4, 5, 6]
    assert ti.slots(b, other, 0, 1) == [13]
    ti.truncate(b, s, 4)
    assert s.block_table == [1] and s.tokens == [1, 2, 3, 4]
    assert b.num_free_pages() == 4
    ti.reserve(b, s, 1)
    assert s.block_table == [1, 2]
    with pytest.raises(ti.OutOfPagesError):
        ti.reserve(b, s, 100)
    assert s.block_table == [1, 2]
    with pytest.raises(ti.ArgumentError):
        ti.truncate(b, s, 10)
    ti.release(b, s)
    ti.release(b, other)
    assert b.num_free_pages() == 6 and s.block_table == []


def test_slots_match_store_formula():
    # slot -> (page, offset) as store_kv! splits it (src/ops/reference.jl:68)
    b = ti.BlockManager(50, 16)
    s = ti.Sequence()
    ti.reserve(b, ti.Sequence(), 40)           # another sequence takes pages 1..3
    ti.reserve(b, s, 100)
    for p, slot in zip(range(0, 100), ti.slots(b, s, 0, 100)):
        assert (slot - 1) // 16 + 1 == s.block_table[p // 16] and (slot - 1) % 16 == p % 16


def test_int8_pools_pairing():
    k, v = ti.int8_kv_pools(64, 4, 2, 5, device="cpu")
    assert k.shape == (5, 2, 4, 64) and k.layer_q.shape == (2, 5, 2, 4, 64)
    assert k.layer_scale.shape == (2, 5, 2, 4)
    lq, ls, sm = ti.layer_arrays(k, v)
    assert lq is k.layer_q and torch.equal(sm, torch.ones(64))
    k2, v2 = ti.int8_kv_pools(64, 4, 2, 5, device="cpu")
    with pytest.raises(ti.ArgumentError):
        ti.layer_arrays(k, v2)
    with pytest.raises(ti.ArgumentError):
        ti.layer_arrays(v, k)


def test_key_smoothing():
    w = torch.tensor([0.5, -2.0, 0.0, 1.0, -1.0, 0.0], dtype=torch.float32)
    assert ti.key_smoothing(w).tolist() == [1.0, 2.0, 1.0, 1.0, 2.0, 1.0]


def test_rotary_table():
    D, L = 128, 40
    t = ti.RotaryTable.build(D, L, 1e6, torch.float32, device="cpu")
    assert t.cos.shape == (L, D) and t.cos_sin.shape == (L, 2, D)
    inv = ti.inverse_frequencies(D, 1e6)
    for p in (0, 1, 39):
        for i in (0, 5, 63):
            ang = np.float32(p) * inv[i]
            assert t.cos[p, i].item() == pytest.approx(math.cos(float(ang)), abs=1e-7)
            assert t.cos[p, i + 64].item() == t.cos[p, i].item()
            assert t.cos_sin[p, 1, i].item() == t.sin[p, i].item()
    assert inv[0] == 1.0 and inv[1] == pytest.approx(1e6 ** (-2 / 128), rel=1e-6)
    # llama3 scaling keeps short wavelengths and divides long ones by `factor`
    sc = ti.Llama3RopeScaling(8.0, 1.0, 4.0, 8192)
    inv3 = ti.inverse_frequencies(D, 5e5, sc)
    base = ti.inverse_frequencies(D, 5e5)
    assert inv3[0] == base[0] and inv3[-1] == pytest.approx(base[-1] / 8, rel=1e-6)


def test_bytes_per_token():
    assert ti.bytes_per_token(36, 8, 128) == 2 * 36 * 8 * 128 * 2
    assert ti.bytes_per_token(36, 8, 128, quantize="int8") == 2 * 36 * 8 * 132
