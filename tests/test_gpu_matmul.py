"""GPU parity of decode-in-matmul against the fp64 oracle (y = x (q - zero)^T scale), tolerance 1e-3 normwise
relative (north star; the kernels reach ~1e-6 because every MFMA product is exact):

  * cf_fused_matmul_async / cf_dense_matmul_async over the reference's single block-Huffman stream: row starts
    inside code blocks (K not a multiple of the block), block sizes 64 / 100 / 37, batches 1..65 (two passes),
    a K beyond one staged 4096-column chunk, a LUT too long for LDS (maxlen 14), a zero point outside the u8 range;
    dense W must hold the reference's exact dequantised values;
  * cf_qw_matmul_async at the C3 shape (4096 x 4096 int4, per-band Huffman or pair-rANS tables, per (row, 64-col)
    scale, bf16 x, B in 1/4/16/64) plus ragged shapes, for both codecs;
  * an identity input (x = I, B = K) through cf_qw_matmul_async gives every dequantised weight bit for bit
    (y[k, m] = (sym[m, k] - zero) * scale[m, k / 64]: one exact product per output), for both codecs.
"""
import numpy as np
import pytest

import oracle as O
from legacy_helpers import huffman_lengths, huffman_stream_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _err(got, ref):
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def _ref_stream(M, K, rng, block, maxlen, bits=4):
    """int4 (or wider) symbols of N(0,1)/sqrt(K) weights, one canonical-Huffman stream, per-tensor scale."""
    W = rng.standard_normal((M, K)) / np.sqrt(K)
    qmax = (1 << (bits - 1)) - 1
    zero = 1 << (bits - 1)
    scale = np.float32(np.abs(W).max() / qmax)
    sym = (np.clip(np.rint(W / scale), -qmax - 1, qmax) + zero).astype(np.int64)
    L = huffman_lengths(np.bincount(sym.ravel(), minlength=1 << bits), maxlen)
    words, boff, lut = huffman_stream_np(sym.ravel(), L, maxlen, block)
    assert np.array_equal(O.huffman_decode(words, lut, maxlen, 0, sym.size), sym.ravel())
    return words, boff, lut, sym, scale, zero


@pytest.mark.parametrize("M,K,B,block,maxlen,zero_shift", [
    (300, 1000, 3, 64, 8, 0), (4096, 4096, 16, 64, 8, 0), (128, 4100, 64, 100, 9, 0), (64, 8192, 65, 64, 8, 0),
    (37, 77, 1, 37, 14, 0), (50, 640, 8, 64, 8, 300)])
def test_reference_stream_fused_and_dense(dev, M, K, B, block, maxlen, zero_shift):
    import torch
    from chromofold_amd import qw
    rng = np.random.default_rng(M + K + B)
    words, boff, lut, sym, scale, zero = _ref_stream(M, K, rng, block, maxlen)
    zero_arg = zero + zero_shift  # an out-of-range zero point shifts every weight by the same constant
    x = rng.standard_normal((B, K)).astype(np.float32)
    ref = O.qmatmul_f64(x, sym, scale, zero_arg)
    d = {k: torch.from_numpy(v.view(np.int32) if v.dtype == np.uint32 else v).to(dev)
         for k, v in (("w", words), ("b", boff), ("l", lut))}
    dx = torch.from_numpy(x).to(dev)
    yf = torch.full((B, M), float("nan"), device=dev)
    qw.fused_matmul(d["w"], d["b"], d["l"], maxlen, block, dx, yf, M, K, float(scale), zero_arg)
    yd = torch.full((B, M), float("nan"), device=dev)
    Wd = torch.empty((M, K), device=dev)
    qw.dense_matmul(d["w"], d["b"], d["l"], maxlen, block, dx, Wd, yd, M, K, float(scale), zero_arg)
    torch.cuda.synchronize()
    exp_w = ((sym - zero_arg).astype(np.float32) * scale).astype(np.float32)
    assert np.array_equal(Wd.cpu().numpy(), exp_w)
    gf, gd = yf.cpu().numpy(), yd.cpu().numpy()
    assert _err(gf, ref) <= 1e-3 and _err(gd, ref) <= 1e-3, (_err(gf, ref), _err(gd, ref))
    assert _err(gf, gd) <= 1e-5


def test_reference_stream_contract(dev):
    from chromofold_amd import _abi
    import torch
    t = torch.zeros(64, device=dev)
    p = t.data_ptr()
    L = _abi.lib()
    assert L.cf_fused_matmul_async(None, p, p, 8, 64, p, p, 1, 1, 1, 1.0, 8, None) == _abi.CF_ERR_INVALID_ARGUMENT
    assert L.cf_fused_matmul_async(p, p, p, 8, 64, p, p, 1, 0, 1, 1.0, 8, None) == _abi.CF_OK  # M == 0
    assert L.cf_dense_matmul_async(p, p, p, 8, 64, p, None, p, 1, 1, 1, 1.0, 8, None) == _abi.CF_ERR_INVALID_ARGUMENT


HUFF, RANS = 1, 2  # CF_QW_CODEC_HUFFMAN, CF_QW_CODEC_RANS


def _qw_check(dev, W, batches, codec=HUFF):
    import torch
    from chromofold_amd import qw
    M, K = W.shape
    h = qw.encode_int4(W, codec)
    mat = qw.QwMatrix(h, dev)
    scales = np.repeat(h.scales, 64, axis=1)[:, :K]
    for B in batches:
        xf = torch.randn((B, K), generator=torch.Generator().manual_seed(B + K)).to(torch.bfloat16)
        x = xf.to(dev)
        y = torch.full((B, M), float("nan"), device=dev)
        mat.matmul_into(x, y)
        torch.cuda.synchronize()
        ref = O.qmatmul_f64(xf.float().numpy(), h.sym, scales, 8)
        e = _err(y.cpu().numpy(), ref)
        assert e <= 1e-3, (B, e)
    return h


@pytest.mark.parametrize("codec", [HUFF, RANS])
@pytest.mark.parametrize("M,K,batches", [(4096, 4096, (1, 4, 16, 64)), (40, 1000, (3, 17)), (24, 8200, (64,)),
                                         (33, 1001, (70, 1)), (20, 12288, (33,))])
def test_qw_matmul(dev, M, K, batches, codec):
    # ragged rows (not a band multiple), K not a multiple of 64 (or of 4: scalar x loads), K over one 4096-column
    # chunk (rANS: a full chunk and a short last one; three full chunks), 70 batch rows (two launches: 4 tiles + 1)
    rng = np.random.default_rng(M * 3 + K)
    _qw_check(dev, rng.standard_normal((M, K)).astype(np.float32), batches, codec)


@pytest.mark.parametrize("codec", [HUFF, RANS])
@pytest.mark.parametrize("M,K", [(512, 4096), (40, 1000), (17, 4160)])
def test_qw_identity_decodes_every_weight(dev, M, K, codec):
    """x = I (B = K rows): y[k, m] = (sym[m, k] - zero) * scale[m, k / 64] is one exact product, so every weight the
    kernel decodes (and its scale) is checked bit for bit against the quantiser's symbols; the weights get a per-row
    spread of magnitudes and a few all-zero segments."""
    import torch
    from chromofold_amd import qw
    rng = np.random.default_rng(M + K + codec)
    W = (rng.standard_normal((M, K)) * np.exp(rng.uniform(-2, 2, (M, 1)))).astype(np.float32)
    W[1, :min(K, 128)] = 0.0
    h = qw.encode_int4(W, codec)
    mat = qw.QwMatrix(h, dev)
    x = torch.eye(K, dtype=torch.bfloat16, device=dev)
    y = torch.full((K, M), float("nan"), device=dev)
    mat.matmul_into(x, y)
    torch.cuda.synchronize()
    want = ((h.sym.astype(np.float32) - 8.0) * np.repeat(h.scales, 64, axis=1)[:, :K]).T
    got = y.cpu().numpy()
    bad = np.argwhere(got != want)
    assert bad.size == 0, (bad[:5], got[tuple(bad[0])], want[tuple(bad[0])])


def test_qw_matmul_skewed_band(dev):
    """A band whose rows differ wildly: 14 zero rows, one two-valued row and one uniform row. The uniform row's
    codes average ~7 bits, more than the kernel stages in LDS per row (640 words per 4096-column chunk), so its
    lanes decode straight from global memory; the other bands take the staged path."""
    rng = np.random.default_rng(99)
    M, K = 48, 4096
    W = np.zeros((M, K), np.float32)
    W[14] = np.where(rng.random(K) < 0.5, -1.0, 1.0)
    W[15] = rng.uniform(-1, 1, K)
    W[16:] = rng.standard_normal((32, K))
    h = _qw_check(dev, W, (1, 16))
    offs = h.offsets.astype(np.int64).ravel()
    ends = np.append(offs[1:], h.words.size * 32).reshape(M, -1)
    first = offs.reshape(M, -1)[:, 0]
    need = (ends[:, -1] >> 5) + 6 - ((first >> 5) & ~3)
    assert need[15] > 640 and need[16:].max() <= 640, need
    _qw_check(dev, W, (1, 16), RANS)  # rANS: the band's table gives the uniform row's pairs ~8 bits each


@pytest.mark.parametrize("codec", [HUFF, RANS])
def test_qw_matmul_graph_replays(dev, codec):
    """cf_qw_matmul_async captured in a HIP graph: every replay (with eager work changing x in between) equals the
    eager call on the same x bit for bit."""
    import torch
    from chromofold_amd import qw
    rng = np.random.default_rng(7)
    M, K, B = 64, 4096, 16
    mat = qw.QwMatrix(qw.encode_int4(rng.standard_normal((M, K)).astype(np.float32), codec), dev)
    x = torch.zeros((B, K), dtype=torch.bfloat16, device=dev)
    y = torch.zeros((B, M), device=dev)
    mat.matmul_into(x, y)  # warm up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        mat.matmul_into(x, y)
    for r in range(3):
        xr = torch.from_numpy(rng.standard_normal((B, K)).astype(np.float32)).to(torch.bfloat16).to(dev)
        x.copy_(xr)
        g.replay()
        torch.cuda.synchronize()
        got = y.clone()
        want = mat.matmul(xr)
        torch.cuda.synchronize()
        assert torch.equal(got, want), r


@pytest.mark.parametrize("codec", [HUFF, RANS])
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_qw_matmul_random_shapes(dev, seed, codec):
    """Random M (not a band multiple), K (ragged last segment, sometimes over one 4096-column chunk) and batch
    (1 .. 140: up to three launches), weights with a per-row spread of magnitudes."""
    rng = np.random.default_rng(1000 + seed)
    M = int(rng.integers(1, 80))
    K = int(rng.integers(1, 9000))
    B = int(rng.integers(1, 141))
    W = (rng.standard_normal((M, K)) * np.exp(rng.uniform(-3, 3, (M, 1)))).astype(np.float32)
    _qw_check(dev, W, (B,), codec)
