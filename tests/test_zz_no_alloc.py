"""cf_kv_paged_attention_batched_noalloc_async (split partials in the library's per-GPU scratch array) against
cf_kv_paged_attention_batched_async (split partials in the caller's workspace): bit-identical outputs on calls in a
row through the C ABI, the second with a smaller input than the first (the scratch array keeps the first call's
partials), a wide-workgroup split, and the size limit (a descriptor whose partials exceed the array is refused before
any launch)."""
import ctypes as C

import numpy as np
import pytest

from kv_helpers import make_seqs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _case(dev, seq_tokens, kv_heads, D, seed, codec=2):
    import torch
    from chromofold_amd import kv
    data = make_seqs(seq_tokens, kv_heads, D, seed)
    tables = None
    if codec == kv.CODEC_RANS_HYBRID:
        parts = []
        n = min(512, seq_tokens[0]) // 16 * 16  # whole pages of sequence 0 sample the tables
        for h in range(kv_heads):
            parts += [kv.build_table(data[0][0][h][:n].reshape(-1, 16, D)),
                      kv.build_table(data[0][1][h][:n].reshape(-1, 16, D))]
        tables = np.concatenate(parts)
    S = len(seq_tokens)
    kvb = kv.build_batched(codec, lambda s: data[s], S, kv_heads, np.array(seq_tokens), D, tables, dev)
    rng = np.random.default_rng(seed + 1)
    q = torch.from_numpy(rng.standard_normal((S, kv_heads * 4, D)).astype(np.float32)).to(dev)
    qp = torch.tensor([t - 1 for t in seq_tokens], dtype=torch.int32, device=dev)
    return kvb, q, qp


def _both(kvb, q, qp, splits):
    """Outputs of the workspace entry point and of the allocation-free one on the same descriptor."""
    import torch
    from chromofold_amd import _abi as A
    L = A.lib()
    L.cf_kv_paged_attention_batched_noalloc_async.restype = C.c_int32
    L.cf_kv_paged_attention_batched_noalloc_async.argtypes = [C.c_void_p, C.c_void_p]
    L.cf_kv_batched_workspace_bytes.restype = C.c_uint64
    sc = 1.0 / np.sqrt(q.shape[2])
    ref = torch.full_like(q, float("nan"))
    kvb.attention(q, ref, qp, sc, splits=splits)
    got = torch.full_like(q, float("nan"))
    d = kvb.desc(q, got, qp, sc, splits=splits)
    need = int(L.cf_kv_batched_workspace_bytes(C.byref(d)))
    d.workspace, d.workspace_bytes = None, 0  # the allocation-free entry point does not read them
    st = L.cf_kv_paged_attention_batched_noalloc_async(C.byref(d), torch.cuda.current_stream().cuda_stream)
    assert st == 0
    torch.cuda.synchronize()
    return ref, got, need


def test_noalloc_matches_workspace_entry_two_calls(dev):
    import torch
    print("case A: 6 seqs x 2 heads, hd 128, splits 3", flush=True)
    kvb, q, qp = _case(dev, [3000, 2500, 1029, 4096, 700, 3333], 2, 128, seed=301)
    ref, got, need = _both(kvb, q, qp, 3)
    assert need > 0
    assert torch.isfinite(ref).all() and torch.equal(ref, got)
    print("case B (smaller): 3 seqs x 1 head, hd 64, splits 2", flush=True)
    kvb2, q2, qp2 = _case(dev, [900, 400, 257], 1, 64, seed=302)
    ref2, got2, need2 = _both(kvb2, q2, qp2, 2)
    assert 0 < need2 < need
    assert torch.isfinite(ref2).all() and torch.equal(ref2, got2)


def test_noalloc_wide_split_and_int8(dev):
    import torch
    print("case C: wide workgroups, 2 splits (>= 96 chain pairs each)", flush=True)
    kvb, q, qp = _case(dev, [13000, 12400], 1, 128, seed=303)
    ref, got, need = _both(kvb, q, qp, 2)
    assert need > 0 and torch.equal(ref, got)
    print("case D: INT8 codec, auto splits", flush=True)
    kvb, q, qp = _case(dev, [500, 1500, 64], 2, 128, seed=304, codec=1)
    ref, got, need = _both(kvb, q, qp, 0)
    assert need > 0 and torch.equal(ref, got)


def test_noalloc_refuses_partials_beyond_the_array(dev):
    import torch
    from chromofold_amd import _abi as A
    L = A.lib()
    L.cf_kv_batched_workspace_bytes.restype = C.c_uint64
    kvb, q, qp = _case(dev, [300, 200], 1, 128, seed=305)
    d = kvb.desc(q, torch.empty_like(q), qp, 0.1, splits=2)
    big = type(d).from_buffer_copy(d)
    big.splits = 64  # 2 x 1 x 64 slots of 4 x 130 floats = 266 KB: fits
    assert L.cf_kv_batched_workspace_bytes(C.byref(big)) <= 8 << 20
    huge = type(d).from_buffer_copy(d)
    # 128 x 64 partial slots (17 MB) exceed the array: refused before any launch (nothing is read)
    huge.seq_count, huge.splits = 128, 64
    assert L.cf_kv_batched_workspace_bytes(C.byref(huge)) > 8 << 20
    L.cf_kv_paged_attention_batched_noalloc_async.restype = C.c_int32
    assert L.cf_kv_paged_attention_batched_noalloc_async(C.byref(huge), None) == A.CF_ERR_UNSUPPORTED
