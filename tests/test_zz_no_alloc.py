"""hq_gqa_decode_noalloc, the attention entry point that allocates nothing
(its workspace is a file-scope device array), against hq_gqa_decode with a
caller workspace: bit-identical outputs on two calls in a row, the second
with a smaller context, through the C ABI.  No reference counterpart: the
variant serves callers that cannot allocate device memory."""
import ctypes

import numpy as np
import pytest

from tests.gpu_util import dev, to_dev, to_host

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _call_both(lib, q, keys, values, context, kv, g, d, capacity, stream):
    out_ws = torch.empty((kv * g, d), dtype=torch.float32, device=dev())
    out_na = torch.full((kv * g, d), float("nan"), dtype=torch.float32, device=dev())
    ws = torch.zeros(lib.hq_gqa_workspace_bytes(capacity, kv, g, d), dtype=torch.uint8, device=dev())
    assert lib.hq_gqa_decode(q.data_ptr(), keys.data_ptr(), values.data_ptr(), ws.data_ptr(), out_ws.data_ptr(),
                             context, kv, g, d, capacity, stream) == 0
    assert lib.hq_gqa_decode_noalloc(q.data_ptr(), keys.data_ptr(), values.data_ptr(), out_na.data_ptr(),
                                     context, kv, g, d, capacity, stream) == 0
    torch.cuda.synchronize()
    return to_host(out_ws), to_host(out_na)


def test_noalloc_first_call_under_graph_capture():
    # The process's first hq_gqa_decode_noalloc call (it takes the array's
    # device address) made inside a HIP graph capture; the graph is replayed
    # three times with new queries written eagerly between the replays, and
    # every replay must equal the workspace entry point's eager result.
    # (This test runs before the file's other no-alloc calls.)
    print("\n[gpu] hq_gqa_decode_noalloc: first call captured in a graph, 3 replays", flush=True)
    from harsh4b_amd import _native
    lib = _native.lib()
    rng = np.random.default_rng(77)
    kv, g, d, capacity, context = 8, 4, 128, 1100, 1000
    keys = to_dev(rng.standard_normal((capacity, kv, d)).astype(np.float16))
    values = to_dev(rng.standard_normal((capacity, kv, d)).astype(np.float16))
    q = torch.empty((kv * g, d), dtype=torch.float32, device=dev())
    out = torch.full((kv * g, d), float("nan"), dtype=torch.float32, device=dev())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    rc = []
    with torch.cuda.graph(graph, stream=s):
        rc.append(lib.hq_gqa_decode_noalloc(q.data_ptr(), keys.data_ptr(), values.data_ptr(), out.data_ptr(),
                                            context, kv, g, d, capacity, ctypes.c_void_p(s.cuda_stream)))
    assert rc == [0]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for rep in range(3):
        q.copy_(to_dev(rng.standard_normal((kv * g, d)).astype(np.float32)))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = to_host(out)
        expect = torch.empty((kv * g, d), dtype=torch.float32, device=dev())
        ws = torch.zeros(lib.hq_gqa_workspace_bytes(capacity, kv, g, d), dtype=torch.uint8, device=dev())
        assert lib.hq_gqa_decode(q.data_ptr(), keys.data_ptr(), values.data_ptr(), ws.data_ptr(),
                                 expect.data_ptr(), context, kv, g, d, capacity, stream) == 0
        assert np.array_equal(got.view(np.uint32), to_host(expect).view(np.uint32)), f"replay {rep}"
        out.fill_(float("nan"))


def test_noalloc_attention_matches_workspace_entry():
    print("\n[gpu] hq_gqa_decode_noalloc vs hq_gqa_decode, contexts 3000 then 70", flush=True)
    from harsh4b_amd import _native
    lib = _native.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rng = np.random.default_rng(1234)
    kv, g, d, capacity = 8, 4, 128, 3100
    keys = to_dev(rng.standard_normal((capacity, kv, d)).astype(np.float16))
    values = to_dev(rng.standard_normal((capacity, kv, d)).astype(np.float16))
    for context in (3000, 70):            # the second call is smaller
        q = to_dev(rng.standard_normal((kv * g, d)).astype(np.float32))
        a, b = _call_both(lib, q, keys, values, context, kv, g, d, capacity, stream)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"context {context}"
    # the largest context the 4 MiB array serves at this head shape, and
    # one past it is refused
    big = 15872
    kb = to_dev(rng.standard_normal((big, kv, d)).astype(np.float16))
    vb = to_dev(rng.standard_normal((big, kv, d)).astype(np.float16))
    q = to_dev(rng.standard_normal((kv * g, d)).astype(np.float32))
    a, b = _call_both(lib, q, kb, vb, big, kv, g, d, big, stream)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "context 15872"
    out = torch.empty((kv * g, d), dtype=torch.float32, device=dev())
    assert lib.hq_gqa_decode_noalloc(q.data_ptr(), kb.data_ptr(), vb.data_ptr(), out.data_ptr(), big + 1, kv, g,
                                     d, big + 1, stream) == 1
