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
    big = 16128
    kb = to_dev(rng.standard_normal((big, kv, d)).astype(np.float16))
    vb = to_dev(rng.standard_normal((big, kv, d)).astype(np.float16))
    q = to_dev(rng.standard_normal((kv * g, d)).astype(np.float32))
    a, b = _call_both(lib, q, kb, vb, big, kv, g, d, big, stream)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "context 16128"
    out = torch.empty((kv * g, d), dtype=torch.float32, device=dev())
    assert lib.hq_gqa_decode_noalloc(q.data_ptr(), kb.data_ptr(), vb.data_ptr(), out.data_ptr(), big + 1, kv, g,
                                     d, big + 1, stream) == 1
