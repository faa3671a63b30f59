"""GPU test of the allocation-free split-KV entry point
(``fl_attn_fwd_f16_splitkv_noalloc``), through the C ABI.

Its partials go to the library's static device scratch array instead of a
caller workspace; the kernels are the same, so its outputs (O and the
log-sum-exp) must equal ``fl_attn_fwd_f16_splitkv``'s bit for bit.  Two calls
in a row, the second on a smaller problem: the array keeps the first call's
partials, so a combine that read a row the second call did not write would
differ.  Both calls are also held to the north_star bound against the fp32
oracle.  A plan whose partials exceed the array is rejected before launch.
"""

import numpy as np
import pytest

from flashlite_amd import capi
from gpu_util import assert_close_oracle, to_dev
from oracle import attention_fp32

pytestmark = pytest.mark.gpu

# (B, H, N_q, N_k, causal, num_splits): the first uses about half the array
# (8 chunks x 32 heads x 64 rows x 272 bytes = 4.5 MB), the second far less.
# The first asks for its 8 chunks explicitly: the library's own plan depends
# on the device's CU count and would run one pass on a partitioned GPU.
CALLS = [(4, 8, 64, 8192, False, 8), (1, 4, 1, 1000, True, 3)]


def _qkv(b, h, nq, nk, seed):
    rs = np.random.RandomState(seed)
    mk = lambda n: rs.standard_normal((b, h, n, 64)).astype(np.float32).astype(np.float16)  # noqa: E731
    return mk(nq), mk(nk), mk(nk)


def _launch(tq, tk, tv, causal, splits, noalloc):
    import torch

    dev = tq.device
    o = torch.full_like(tq, float("nan"))
    ls = torch.full(tq.shape[:3], float("nan"), dtype=torch.float32, device=dev)
    p = capi.tensor_params_ex(tq, tk, tv, o, 0.125, causal, lse=ls)
    stream = torch.cuda.current_stream(dev).cuda_stream
    need = capi.splitkv_workspace_bytes(p, splits)
    assert 0 < need <= capi.SCRATCH_BYTES, need
    if noalloc:
        capi.check(capi.fwd_splitkv_noalloc(p, stream, splits))
    else:
        ws = torch.full((need // 4,), float("nan"), dtype=torch.float32, device=dev)
        capi.check(capi.fwd_splitkv(p, ws.data_ptr(), need, stream, splits))
    torch.cuda.synchronize(dev)
    return o, ls


def test_noalloc_matches_workspace_entry_point(cuda):
    import torch

    for i, (b, h, nq, nk, causal, splits) in enumerate(CALLS):
        print(f"noalloc call {i}: B{b} H{h} Nq{nq} Nk{nk} causal={causal} splits={splits}",
              flush=True)
        q16, k16, v16 = _qkv(b, h, nq, nk, seed=100 + i)
        tq, tk, tv = (to_dev(x, cuda) for x in (q16, k16, v16))
        o_ws, l_ws = _launch(tq, tk, tv, causal, splits, noalloc=False)
        o_na, l_na = _launch(tq, tk, tv, causal, splits, noalloc=True)
        assert torch.equal(o_na, o_ws), f"call {i}: O differs from the workspace entry point"
        assert torch.equal(l_na, l_ws), f"call {i}: lse differs from the workspace entry point"
        assert_close_oracle(o_na.float().cpu().numpy(), q16, k16, v16, 0.125, causal,
                            ref=attention_fp32(q16, k16, v16, 0.125, causal))


def test_noalloc_rejects_oversized_plan(cuda):
    import torch

    # 16 chunks x 64 heads x 256 rows x 272 bytes = 71 MB of partials
    tq = torch.zeros((4, 16, 256, 64), dtype=torch.float16, device=cuda)
    tk = torch.zeros((4, 16, 4096, 64), dtype=torch.float16, device=cuda)
    o = torch.full_like(tq, 7.0)
    p = capi.tensor_params_ex(tq, tk, tk, o, 0.125, False)
    assert capi.splitkv_workspace_bytes(p, 16) > capi.SCRATCH_BYTES
    rc = capi.fwd_splitkv_noalloc(p, torch.cuda.current_stream(cuda).cuda_stream, 16)
    assert rc == capi.FL_ERR_UNSUPPORTED
    assert "scratch" in capi.last_error()
    torch.cuda.synchronize(cuda)
    assert bool((o == 7.0).all()), "a rejected call launched work"


# The library's own plan (num_splits = 0) lowered to fit the array:
# (B, H, N_q, N_k, chunks with a workspace, chunks without). B4 H16 N_q 128
# over 1024 keys plans 4 chunks of 64 groups (8.9 MB) and runs 3; B4 H31
# N_q 128 over 4096 keys plans 3 chunks (12.9 MB) and runs one pass; B2 H16
# N_q 128 over 4096 keys plans 8 chunks of 32 groups (8.9 MB) and runs 7.
CAPPED = [(4, 16, 128, 1024, 4, 3), (4, 31, 128, 4096, 3, 0), (2, 16, 128, 4096, 8, 7)]


@pytest.mark.parametrize("b,h,nq,nk,ws_chunks,na_chunks", CAPPED)
def test_noalloc_library_plan_is_capped(cuda, b, h, nq, nk, ws_chunks, na_chunks):
    import torch

    print(f"capped plan: B{b} H{h} Nq{nq} Nk{nk}", flush=True)
    if _cus(cuda) != 256:
        pytest.skip("the plans below are the whole MI355X's (256 CUs)")
    q16, k16, v16 = _qkv(b, h, nq, nk, seed=7)
    tq, tk, tv = (to_dev(x, cuda) for x in (q16, k16, v16))
    o = torch.full_like(tq, float("nan"))
    ls = torch.full(tq.shape[:3], float("nan"), dtype=torch.float32, device=cuda)
    p = capi.tensor_params_ex(tq, tk, tv, o, 0.125, False, lse=ls)
    per_chunk = b * h * nq * 68 * 4
    assert capi.splitkv_workspace_bytes(p, 0) == ws_chunks * per_chunk > capi.SCRATCH_BYTES
    assert capi.splitkv_noalloc_bytes(p, 0) == na_chunks * per_chunk
    stream = torch.cuda.current_stream(cuda).cuda_stream
    capi.check(capi.fwd_splitkv_noalloc(p, stream, 0))
    torch.cuda.synchronize(cuda)
    # the same plan through the other entry points, bit for bit
    o2 = torch.full_like(tq, float("nan"))
    l2 = torch.full(tq.shape[:3], float("nan"), dtype=torch.float32, device=cuda)
    p2 = capi.tensor_params_ex(tq, tk, tv, o2, 0.125, False, lse=l2)
    if na_chunks == 0:
        capi.check(capi.fwd_ex(p2, stream))
    else:
        need = capi.splitkv_workspace_bytes(p2, na_chunks)
        assert need == na_chunks * per_chunk
        ws = torch.full((need // 4,), float("nan"), dtype=torch.float32, device=cuda)
        capi.check(capi.fwd_splitkv(p2, ws.data_ptr(), need, stream, na_chunks))
    torch.cuda.synchronize(cuda)
    assert torch.equal(o, o2) and torch.equal(ls, l2)
    hs = slice(0, 2)  # two heads of the first batch against the oracle
    assert_close_oracle(o[:1, hs].float().cpu().numpy(), q16[:1, hs], k16[:1, hs], v16[:1, hs],
                        0.125, False)


def _cus(dev):
    import torch

    return torch.cuda.get_device_properties(dev).multi_processor_count


def test_noalloc_under_graph_capture(cuda):
    """One eager call (the first call per device looks the scratch address
    up), then two allocation-free calls captured in a HIP graph and replayed
    several times, with eager work and synchronisation between replays:
    every replay equals the eager outputs bit for bit."""
    import torch

    shapes = [(2, 8, 1, 4096, True, 8), (4, 8, 32, 2048, False, 4)]
    data, eager = [], []
    stream = torch.cuda.Stream(cuda)
    for i, (b, h, nq, nk, causal, splits) in enumerate(shapes):
        print(f"graph call {i}: B{b} H{h} Nq{nq} Nk{nk} causal={causal} splits={splits}",
              flush=True)
        q16, k16, v16 = _qkv(b, h, nq, nk, seed=40 + i)
        tq, tk, tv = (to_dev(x, cuda) for x in (q16, k16, v16))
        o = torch.full_like(tq, float("nan"))
        ls = torch.full(tq.shape[:3], float("nan"), dtype=torch.float32, device=cuda)
        p = capi.tensor_params_ex(tq, tk, tv, o, 0.125, causal, lse=ls)
        assert 0 < capi.splitkv_noalloc_bytes(p, splits) <= capi.SCRATCH_BYTES
        with torch.cuda.stream(stream):
            capi.check(capi.fwd_splitkv_noalloc(p, stream.cuda_stream, splits))
        stream.synchronize()
        eager.append((o.clone(), ls.clone()))
        o.fill_(float("nan"))
        ls.fill_(float("nan"))
        # the params hold raw addresses: keep the tensors alive for the graph
        # (torch.cuda.graph empties the caching allocator on entry, which
        # would unmap the memory of tensors that are no longer referenced)
        data.append((p, o, ls, splits, (q16, k16, v16, causal), (tq, tk, tv)))
    torch.cuda.synchronize(cuda)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for p, _, _, splits, _, _ in data:
            capi.check(capi.fwd_splitkv_noalloc(p, stream.cuda_stream, splits))
    for rep in range(3):
        for _, o, ls, _, _, _ in data:
            o.fill_(float("nan"))
            ls.fill_(float("nan"))
        junk = torch.randn(1 << 20, device=cuda) * 2.0  # eager work between replays
        torch.cuda.synchronize(cuda)
        graph.replay()
        torch.cuda.synchronize(cuda)
        assert bool(torch.isfinite(junk).all())
        for i, (_, o, ls, _, _, _) in enumerate(data):
            assert torch.equal(o, eager[i][0]), f"replay {rep}, call {i}: O differs from eager"
            assert torch.equal(ls, eager[i][1]), f"replay {rep}, call {i}: lse differs from eager"
    q16, k16, v16, causal = data[0][4]
    assert_close_oracle(data[0][1].float().cpu().numpy(), q16, k16, v16, 0.125, causal)
