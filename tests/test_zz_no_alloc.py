"""ti_attention_noalloc (split-KV partials in the library's static device scratch, no
allocation) against ti_attention with a caller workspace, through the C ABI: the same
kernels and plan, so outputs must be bit-identical. Each case makes two calls in a row on
the same GPU, the second with a smaller input, and checks both (the scratch keeps the
first call's contents); the first output is also checked against the oracle."""
import ctypes
import math

import numpy as np
import pytest
import torch

import tileinfer_hip as ti
from tileinfer_hip import _lib
from tileinfer_hip.backend import _attention_args, _stream, kv_cache_struct
from helpers import randn, rng
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
BE = ti.HipBackend()

# (name, kind, Hq, Hk, P, [(B, start, n), (B, start, n)] first call, second call, path)
CASES = [
    ("decode_b1_splits", "bf16", 32, 8, 16, [(1, 4095, 1), (1, 999, 1)], _lib.TI_PATH_AUTO),
    ("decode_b32_nows", "bf16", 32, 8, 16, [(32, 2047, 1), (32, 500, 1)], _lib.TI_PATH_AUTO),
    ("verify", "bf16", 32, 8, 16, [(16, 4096, 16), (4, 1000, 16)], _lib.TI_PATH_AUTO),
    ("prefill_pp_splits", "bf16", 8, 1, 16, [(1, 0, 256), (1, 0, 100)], _lib.TI_PATH_PREFILL_PINGPONG),
    ("prefill_4w_splits", "bf16", 32, 8, 16, [(1, 1024, 64), (1, 300, 40)], _lib.TI_PATH_PREFILL_DIRECT),
    ("decode_int8", "int8", 32, 8, 16, [(2, 3000, 1), (2, 700, 1)], _lib.TI_PATH_AUTO),
    # fp32 on the matrix-core decode kernel (16-token pages; the second call has fewer active
    # splits), and on the VALU kernel (8-token pages)
    ("fp32_mfma", "fp32", 16, 8, 16, [(1, 4095, 1), (1, 200, 1)], _lib.TI_PATH_AUTO),
    ("generic_fp32", "fp32", 16, 8, 8, [(1, 1023, 1), (1, 200, 1)], _lib.TI_PATH_AUTO),
    # split batches shared out by length (flat mode) and the 16-row paired prefill (bf16, INT8)
    ("decode_flat", "bf16", 32, 8, 16, [(6, 3000, 1), (4, 700, 1)], _lib.TI_PATH_AUTO),
    ("prefill_paired16", "bf16", 32, 8, 16, [(1, 0, 512), (1, 1024, 128)], _lib.TI_PATH_AUTO),
    ("prefill_paired16_int8", "int8", 32, 8, 16, [(1, 0, 512), (1, 300, 200)], _lib.TI_PATH_AUTO),
    # the ping-pong kernel pinned on 512 tokens of one KV head with G = 8: its split partials
    # (16 x 4096 rows) exceed the scratch, so noalloc runs it unsplit, as ti_attention does
    # without a workspace; the second call fits the scratch and splits
    ("prefill_pp_over_scratch", "bf16", 8, 1, 16, [(1, 0, 512), (1, 0, 256)], _lib.TI_PATH_PREFILL_PINGPONG),
]


def _inputs(g, kind, Hq, Hk, P, B, start, n, D=128):
    L = start + n
    per = -(-L // P)
    pages = B * per + 3
    perm = g.permutation(pages)[:B * per] + 1
    bts = perm.reshape(B, per).astype(np.int32)
    bf16 = kind != "fp32"
    q = randn(g, B * n, Hq, D, bf16=bf16)
    dtype = torch.float32 if kind == "fp32" else torch.bfloat16
    qd = torch.from_numpy(q).to(dtype).cuda()
    if kind == "int8":
        kq, vq = ti.int8_kv_pools(D, P, Hk, pages)
        kq.layer_q.copy_(torch.from_numpy(g.integers(-127, 128, kq.layer_q.shape).astype(np.int8)))
        kq.layer_scale.copy_(torch.from_numpy(g.random(kq.layer_scale.shape, dtype=np.float32) * 0.02 + 0.001))
        k, v = kq, vq
        ref_kw = dict(layer_q=kq.layer_q.cpu().numpy(), layer_scale=kq.layer_scale.cpu().numpy(),
                      smooth=kq.smooth.cpu().numpy())
    else:
        kp, vp = randn(g, pages, Hk, P, D, bf16=bf16), randn(g, pages, Hk, P, D, bf16=bf16)
        k, v = torch.from_numpy(kp).to(dtype).cuda(), torch.from_numpy(vp).to(dtype).cuda()
        ref_kw = dict(k_pages=kp, v_pages=vp)
    pos = torch.arange(start, L, dtype=torch.int32).repeat(B).cuda()
    return dict(q=q, qd=qd, k=k, v=v, bts=bts, btd=torch.from_numpy(bts).cuda(), pos=pos, B=B, n=n,
                start=start, ref_kw=ref_kw)


def _call(fn_name, x, path, workspace):
    out = torch.full_like(x["qd"], float("nan"))
    a = _attention_args(out, x["qd"], x["btd"], x["pos"], 1 / math.sqrt(128), True, path, x["B"], x["n"],
                        None, workspace)
    c = kv_cache_struct(x["k"], x["v"])
    st = getattr(_lib.load(), fn_name)(ctypes.byref(a), ctypes.byref(c), _stream(x["qd"]))
    assert st == _lib.TI_OK, f"{fn_name}: status {st}"
    return out


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_noalloc_matches_attention(gpu, case):
    name, kind, Hq, Hk, P, calls, path = case
    g = rng(5100 + len(name))
    for i, (B, start, n) in enumerate(calls):
        print(f"noalloc {name} call {i}: B={B} start={start} n={n} path={path}", flush=True)
        x = _inputs(g, kind, Hq, Hk, P, B, start, n)
        ws = ti.attention_workspace(BE, x["qd"], x["k"], num_seqs=B, max_query_len=n, path=path)
        if ws is not None and ws.numel() > _lib.NOALLOC_SCRATCH_BYTES:
            ws = None                               # noalloc runs this shape unsplit
        want = _call("ti_attention", x, path, ws)
        got = _call("ti_attention_noalloc", x, path, None)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {i}: differs from ti_attention"
        if i == 0 and ws is not None:
            assert ws.numel() > 0                   # this case does use split partials
        got_h = got.float().cpu().numpy()
        tol = 1e-4 if kind == "fp32" else 2e-2
        for b in range(min(B, 2)):
            ref = orc.attention(x["q"][b * n:(b + 1) * n], x["bts"][b], start, 1 / math.sqrt(128), True,
                                **x["ref_kw"])
            err = float(np.max(np.abs(ref - got_h[b * n:(b + 1) * n])))
            assert err <= tol, f"call {i} seq {b}: max abs err {err}"


@pytest.mark.parametrize("case", [CASES[0], CASES[2], CASES[8]], ids=lambda c: c[0])
def test_noalloc_allocates_nothing_and_replays_in_a_graph(gpu, case):
    """The defining property: no allocation. The eager call leaves torch's allocator
    untouched, and the call captured in a HIP graph replays (several times, with eager work
    and synchronizations between the replays) to the eager output bit for bit."""
    name, kind, Hq, Hk, P, calls, path = case
    g = rng(5300 + len(name))
    B, start, n = calls[0]
    print(f"noalloc graph {name}: B={B} start={start} n={n}", flush=True)
    x = _inputs(g, kind, Hq, Hk, P, B, start, n)
    out = torch.full_like(x["qd"], float("nan"))
    a = _attention_args(out, x["qd"], x["btd"], x["pos"], 1 / math.sqrt(128), True, path, B, n, None, None)
    c = kv_cache_struct(x["k"], x["v"])
    L = _lib.load()
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    assert L.ti_attention_noalloc(ctypes.byref(a), ctypes.byref(c), _stream(x["qd"])) == _lib.TI_OK
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = L.ti_attention_noalloc(ctypes.byref(a), ctypes.byref(c), _stream(x["qd"]))
    assert st == _lib.TI_OK
    for r in range(4):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r} differs from the eager call"
        x["qd"].mul_(1.0)                           # eager work between replays
        torch.cuda.synchronize()
