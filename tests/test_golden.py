"""The oracle against the committed golden fixtures (tests/golden/, written by
tests/golden/make_golden.py): the stored outputs are reproduced from the stored inputs,
so an accidental change to the oracle shows up here, without a GPU."""
import math
import os
import sys

import numpy as np

from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_golden  # noqa: E402


def load(name):
    return np.load(os.path.join(GOLDEN, name))


def test_attention_bf16_fixture():
    f = load("attention_bf16.npz")
    for causal, key in ((True, "out_causal"), (False, "out_noncausal")):
        out = orc.attention(f["q"], f["block_table"], int(f["start"]), float(f["scale"]), causal,
                            f["k_pages"], f["v_pages"])
        assert np.array_equal(out, f[key]), key
    # the two masks differ: the last query sees every key either way, the first does not
    assert np.array_equal(f["out_causal"][-1], f["out_noncausal"][-1])
    assert not np.allclose(f["out_causal"][0], f["out_noncausal"][0])


def test_attention_int8_fixture():
    f = load("attention_int8.npz")
    out = orc.attention(f["q"], f["block_table"], int(f["start"]), float(f["scale"]), True,
                        layer_q=f["layer_q"], layer_scale=f["layer_scale"], smooth=f["smooth"])
    assert np.array_equal(out, f["out"])


def test_store_kv_int8_fixture():
    f = load("store_kv_int8.npz")
    lq = np.zeros_like(f["layer_q"])
    ls = np.zeros_like(f["layer_scale"])
    orc.store_kv_int8(lq, ls, f["smooth"], f["k"], f["v"], f["slots"])
    assert np.array_equal(lq, f["layer_q"]) and np.array_equal(ls, f["layer_scale"])
    # the stored cases: a zero value vector quantizes to 0 with scale 0, the halfway
    # value 0.5 * 127 / 127 + 1/2 = 1 rounds up
    P = f["layer_q"].shape[3]
    s = int(f["slots"][3]) - 1
    vq, vs = f["layer_q"][1, s // P, 1, s % P], f["layer_scale"][1, s // P, 1, s % P]
    assert vq[0] == 127 and vq[1] == 1 and vs == np.float32(1.0)


def test_attention_inputs_fixture():
    f = load("attention_inputs.npz")
    kp = np.zeros_like(f["k_pages"])
    vp = np.zeros_like(f["v_pages"])
    nq = f["q"].shape[1]
    nkv = f["k_pages"].shape[1]
    q = orc.attention_inputs(f["qkv"], f["q_norm"], f["k_norm"], f["cos_sin"], f["positions"], f["slots"],
                             nq, nkv, float(f["eps"]), True, k_pages=kp, v_pages=vp)
    assert np.array_equal(q, f["q"])
    assert np.array_equal(kp, f["k_pages"]) and np.array_equal(vp, f["v_pages"])


def test_config1_fixture():
    f = load("config1_fp32.npz")
    q, k, v, bt = make_golden.config1_pools(int(f["seed"]))
    assert np.array_equal(make_golden.digest(k, v), f["pools_sha256"]), "pool generation changed"
    assert np.array_equal(q, f["q"]) and np.array_equal(bt, f["block_table"])
    out = orc.attention(q, bt, int(f["start"]), float(f["scale"]), True, k, v)
    assert np.array_equal(out, f["out"])
    assert math.isclose(float(f["scale"]), 1 / math.sqrt(128), rel_tol=1e-7)
