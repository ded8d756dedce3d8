"""The HIP kernels against the committed golden fixtures (tests/golden/): stored inputs
in, stored oracle outputs compared. Tolerances: max abs <= 2e-2 (bf16, INT8-KV) and
<= 1e-4 (fp32) against the double-accumulated oracle; the INT8 store and the fused
RoPE + KV write bit-exact."""
import os
import sys

import numpy as np
import pytest
import torch

import tileinfer_hip as ti
from helpers import ulps

pytestmark = pytest.mark.gpu
BE = ti.HipBackend()
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_golden  # noqa: E402


def load(name):
    return np.load(os.path.join(GOLDEN, name))


def dev(x, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x))
    return (t.to(dtype) if dtype is not None else t).cuda()


@pytest.mark.parametrize("path", [ti.TI_PATH_AUTO, ti.TI_PATH_DECODE, ti.TI_PATH_PREFILL])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_bf16_golden(gpu, path, causal):
    f = load("attention_bf16.npz")
    q = dev(f["q"], torch.bfloat16)
    k, v = dev(f["k_pages"], torch.bfloat16), dev(f["v_pages"], torch.bfloat16)
    n = q.shape[0]
    pos = torch.arange(int(f["start"]), int(f["start"]) + n, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    ws = ti.attention_workspace(BE, q, k, path=path)
    ti.attention_(BE, out, ws, q, k, v, dev(f["block_table"]), pos, float(f["scale"]), causal, path=path)
    ref = f["out_causal" if causal else "out_noncausal"]
    got = out.float().cpu().numpy()
    assert float(np.max(np.abs(ref - got))) <= 2e-2
    assert ulps(ref, got) <= 5


def test_attention_int8_golden(gpu):
    f = load("attention_int8.npz")
    _, pages, Hk, P, D = f["layer_q"].shape
    kq, vq = ti.int8_kv_pools(D, P, Hk, pages, key_smoothing=torch.from_numpy(f["smooth"]))
    kq.layer_q.copy_(dev(f["layer_q"]))
    kq.layer_scale.copy_(dev(f["layer_scale"]))
    q = dev(f["q"], torch.bfloat16)
    n = q.shape[0]
    pos = torch.arange(int(f["start"]), int(f["start"]) + n, dtype=torch.int32, device="cuda")
    for path in (ti.TI_PATH_AUTO, ti.TI_PATH_PREFILL):
        out = torch.empty_like(q)
        ws = ti.attention_workspace(BE, q, kq, path=path)
        ti.attention_(BE, out, ws, q, kq, vq, dev(f["block_table"]), pos, float(f["scale"]), True, path=path)
        assert float(np.max(np.abs(f["out"] - out.float().cpu().numpy()))) <= 2e-2


def test_store_kv_int8_golden(gpu):
    f = load("store_kv_int8.npz")
    _, pages, Hk, P, D = f["layer_q"].shape
    kq, vq = ti.int8_kv_pools(D, P, Hk, pages, key_smoothing=torch.from_numpy(f["smooth"]))
    ti.store_kv_(BE, kq, vq, dev(f["k"], torch.bfloat16), dev(f["v"], torch.bfloat16), dev(f["slots"]))
    assert np.array_equal(kq.layer_q.cpu().numpy(), f["layer_q"])
    assert np.array_equal(kq.layer_scale.cpu().numpy(), f["layer_scale"])


def test_attention_inputs_golden(gpu):
    f = load("attention_inputs.npz")
    nq, nkv = f["q"].shape[1], f["k_pages"].shape[1]
    table = ti.RotaryTable.from_arrays(torch.from_numpy(f["cos_sin"][:, 0]), torch.from_numpy(f["cos_sin"][:, 1]),
                                       torch.bfloat16)
    k = torch.zeros(f["k_pages"].shape, dtype=torch.bfloat16, device="cuda")
    v = torch.zeros_like(k)
    q = torch.empty(f["q"].shape, dtype=torch.bfloat16, device="cuda")
    ti.attention_inputs_(BE, q, k, v, dev(f["qkv"], torch.bfloat16), dev(f["q_norm"], torch.bfloat16),
                         dev(f["k_norm"], torch.bfloat16), table, dev(f["positions"]), dev(f["slots"]),
                         float(f["eps"]))
    assert np.array_equal(q.float().cpu().numpy(), f["q"])
    assert np.array_equal(k.float().cpu().numpy(), f["k_pages"])
    assert np.array_equal(v.float().cpu().numpy(), f["v_pages"])
    assert nq == 4 and nkv == 2


def test_config1_fp32_golden(gpu):
    f = load("config1_fp32.npz")
    q, k, v, bt = make_golden.config1_pools(int(f["seed"]))
    assert np.array_equal(make_golden.digest(k, v), f["pools_sha256"])
    qd = dev(q)
    pos = torch.tensor([int(f["start"])], dtype=torch.int32, device="cuda")
    out = ti.attention(BE, qd, dev(k), dev(v), dev(bt), pos, float(f["scale"]))
    assert float(np.max(np.abs(f["out"] - out.cpu().numpy()))) <= 1e-4
