"""Host side of the batched attention runtime (cf_attention_runtime_*, reference include/chromofold/
production_attention.h) and the pinning of its CPU oracle (oracle.rt_*), no device work.

The oracle restates reference src/cuda/production_attention.cu:59-139. It is pinned by:
  * the nibble decode against sign extension by arithmetic shift (an independent form of the two's-complement
    rule), for every byte value;
  * the per-row block layout by the quantiser round trip (|x - dequant| <= scale / 2 for every value, with
    head_dim not a multiple of the block size, where a flat block index would break the bound);
  * its attention against the pinned sealed-page oracle (oracle.nib_attention) on the same pages, nibbles
    converted offset-8 -> two's complement by xor 8, where the two formats and visibility rules coincide;
  * the visibility rule (no causal bound, inclusive window) by closed forms: with K = 0 the output is the mean of
    the V rows of exactly the listed positions;
  * NULL pages skipped and an empty item giving zeros.
"""
import numpy as np
import pytest

import oracle as O
from chromofold_amd import sealkv as S


def test_nibble_decode_is_twos_complement():
    b = np.arange(256, dtype=np.uint8)
    got = O.rt_dequant(b, np.ones(1, np.float32), 1, 1, 512, 512, 512).ravel()
    lo = (b.astype(np.int8) << 4).astype(np.int8) >> 4  # sign-extend the low nibble by arithmetic shift
    hi = b.astype(np.int8) >> 4
    assert np.array_equal(got[0::2], lo.astype(np.float64))
    assert np.array_equal(got[1::2], hi.astype(np.float64))


@pytest.mark.parametrize("D,bs", [(40, 16), (64, 24), (128, 32), (8, 64), (96, 7)])
def test_row_block_round_trip(D, bs):
    rng = np.random.default_rng(D + bs)
    T, H = 9, 3
    x = (rng.standard_normal((T, H, D)) * rng.uniform(0.01, 50, (T, H, 1))).astype(np.float32)
    x[0, 1] = 0.0  # an all-zero row: scale 1, values 0
    payload, scales = O.rt_quantize(x, bs)
    bpr = -(-D // bs)
    assert scales.shape == (T * H * bpr,) and payload.shape == ((T * H * D + 1) // 2,)
    got = O.rt_dequant(payload, scales, T, H, D, D, bs)
    sc = np.repeat(scales.reshape(T, H, bpr), bs, axis=2)[:, :, :D].astype(np.float64)
    assert np.all(np.abs(got - x) <= sc / 2 + 1e-6 * np.abs(x))
    # the block maximum lands on +-7 exactly: the scale is absmax / 7
    blocks = np.zeros((T, H, bpr * bs))
    blocks[:, :, :D] = np.abs(x)
    amax = blocks.reshape(T, H, bpr, bs).max(axis=3).ravel()
    nz = amax > 0
    assert np.allclose(scales[nz], amax[nz] / 7, rtol=1e-6) and np.all(scales[~nz] == 1)


@pytest.mark.parametrize("kvh,gqa,D,bs", [(2, 4, 64, 32), (1, 1, 128, 128), (3, 2, 32, 16)])
def test_attention_equals_sealed_page_oracle(kvh, gqa, D, bs):
    """Sealed pages (offset-8 symbols, blocks over the page's flat values) xor 8 are runtime pages when the block
    size divides head_dim; with every position before the query and no window both rules see every token."""
    rng = np.random.default_rng(kvh * 100 + D)
    page, npages = 16, 4
    K = rng.standard_normal((npages * page, kvh, D)).astype(np.float32)
    V = rng.standard_normal((npages * page, kvh, D)).astype(np.float32)
    sealed, runtime = [], []
    for p in range(npages):
        sp = O.nib_seal_page(K[p * page:(p + 1) * page], V[p * page:(p + 1) * page], p * page, bs)
        sealed.append(sp)
        runtime.append(O.RtPage(sp.k_payload ^ np.uint8(0x88), sp.v_payload ^ np.uint8(0x88), sp.k_scales,
                                sp.v_scales, p * page, page, D, bs))
    ak = rng.standard_normal((5, kvh, D)).astype(np.float32)
    av = rng.standard_normal((5, kvh, D)).astype(np.float32)
    q = rng.standard_normal((kvh * gqa, D)).astype(np.float32)
    qpos = npages * page + 10
    want = O.nib_attention(sealed, bs, q[None], qpos, kvh, gqa, 0.2, 0, ak, av, npages * page)[0]
    got = O.rt_attention_f64(q, kvh, gqa, qpos, 0, 0.2, runtime, ak, av, npages * page)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def _k_zero_pages(positions, kvh, D, bs):
    """One runtime page per position: K = 0 (all scores equal) and V rows all equal to the position."""
    pages = []
    for p in positions:
        kp, ks = O.rt_quantize(np.zeros((1, kvh, D), np.float32), bs)
        vp, vs = O.rt_quantize(np.full((1, kvh, D), 7.0, np.float32), bs)  # nibble 7 with scale 1
        pages.append(O.RtPage(kp, vp, ks, vs * np.float32(p / 7.0), p, 1, D, bs))
    return pages


@pytest.mark.parametrize("qpos,window,visible", [
    (10, 0, list(range(0, 20))),          # no window: every position, the 9 after the query included
    (10, 3, list(range(7, 20))),          # p + 3 >= 10: 7 is in (inclusive bound), 6 is out
    (10, 10, list(range(0, 20))),
    (10, 11, list(range(0, 20))),
    (2, 1, list(range(1, 20))),
    (25, 4, []),                          # nothing within the window: zeros
])
def test_visibility_closed_form(qpos, window, visible):
    kvh, D, bs = 2, 16, 8
    pages = _k_zero_pages(range(20), kvh, D, bs)
    q = np.ones((kvh, D), np.float32)
    got = O.rt_attention_f64(q, kvh, 1, qpos, window, 1.0, pages)
    want = np.mean(visible) if visible else 0.0
    assert np.allclose(got, want, rtol=1e-6, atol=0)  # the V scales p / 7 are fp32


def test_null_pages_skipped_and_empty_item():
    kvh, D, bs = 1, 16, 8
    pages = _k_zero_pages([1, 2, 3], kvh, D, bs)
    holed = [pages[0], O.RtPage(None, pages[1].v_payload, pages[1].k_scales, pages[1].v_scales, 2, 1, D, bs), pages[2]]
    q = np.ones((1, D), np.float32)
    assert np.allclose(O.rt_attention_f64(q, kvh, 1, 5, 0, 1.0, holed), 2.0)  # mean of 1 and 3
    assert not O.rt_attention_f64(q, kvh, 1, 5, 0, 1.0, []).any()


# ------------------------------------------------------------------------------------------- host contract
def test_runtime_contract_without_device_work():
    with pytest.raises(S.SealError):
        S.AttentionRuntime(1, 2, 6, 64, gqa=4)  # 6 != 2 * 4
    with pytest.raises(S.SealError):
        S.AttentionRuntime(1, 2, 8, 60)  # head_dim not a multiple of 8
    with pytest.raises(S.SealError):
        S.AttentionRuntime(0, 2, 8, 64)
    rt = S.AttentionRuntime(1, 2, 8, 64, mode=S.CF_ATTENTION_REFERENCE)
    items = (S.cf_attention_batch_item * 2)()
    assert rt.execute_items(items) == -1 and "OPTIMIZED" in rt.last_error()
    assert rt.counters()["reference_launches"] == 1
    rt.close()
    rt = S.AttentionRuntime(1, 2, 8, 64)
    assert rt.execute_items(items) == -1 and "NULL" in rt.last_error()
    c = rt.counters()
    assert c["optimized_launches"] == 0 and c["cuda_errors"] == 0 and c["allocation_count"] == 0
    rt.close()
