"""The measurement kernels of chromofold_measure.h on the GPU.

cf_stream_read_async reads every byte once, one workgroup per 64 KiB chunk, and stores a chunk's XOR fold (of its
32-bit words) to the sink only when it equals CF_MEASURE_FOLD_KEY. Buffers built so that exactly one chunk folds to
the key check the chunking, the ragged last chunk and that no other chunk's fold lands in the sink."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

KEY = 0x2545F491  # CF_MEASURE_FOLD_KEY
CHUNK = 65536


@pytest.fixture(scope="module")
def lib():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from chromofold_amd import _abi as A
    A.declare("cf_stream_read_async", A.I32, [A.P, A.U64, A.P, A.P])
    A.declare("cf_cache_read_async", A.I32, [A.P, A.U64, A.U32, A.P, A.P])
    A.declare("cf_lds_read_async", A.I32, [A.U32, A.P, A.P])
    return A


def _stream(A, words: np.ndarray) -> int:
    import torch
    buf = torch.from_numpy(words.view(np.int32)).to("cuda:0")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    A.check(A.lib().cf_stream_read_async(buf.data_ptr(), words.nbytes, sink.data_ptr(), None), "cf_stream_read_async")
    torch.cuda.synchronize()
    return int(sink.cpu().numpy().view(np.uint32)[0])


def _with_fold(words: np.ndarray, lo: int, hi: int, target: int) -> None:
    """Adjust words[hi - 1] so that the XOR of words[lo:hi] is `target`."""
    words[hi - 1] ^= np.uint32(np.bitwise_xor.reduce(words[lo:hi]) ^ target)


@pytest.mark.parametrize("nbytes, key_chunk", [(16, 0), (CHUNK, 0), (CHUNK + 16, 1), (3 * CHUNK + 48, 3),
                                               (5 * CHUNK, 2), (1 << 24, 200)])
def test_stream_read_folds_each_chunk_once(lib, nbytes, key_chunk):
    rng = np.random.default_rng(nbytes)
    words = rng.integers(0, 1 << 32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
    per = CHUNK // 4
    nchunks = (len(words) + per - 1) // per
    for c in range(nchunks):  # every other chunk folds to something else than the key
        lo, hi = c * per, min((c + 1) * per, len(words))
        _with_fold(words, lo, hi, KEY ^ 0x1 if c != key_chunk else KEY)
    assert _stream(lib, words) == KEY
    lo, hi = key_chunk * per, min((key_chunk + 1) * per, len(words))
    _with_fold(words, lo, hi, KEY ^ 0x80000000)  # now no chunk folds to the key: the sink stays 0
    assert _stream(lib, words) == 0


def test_stream_read_argument_rules(lib):
    import torch
    A = lib
    buf = torch.zeros(64, dtype=torch.int32, device="cuda:0")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    L = A.lib()
    assert L.cf_stream_read_async(buf.data_ptr(), 0, sink.data_ptr(), None) == A.CF_OK
    assert L.cf_stream_read_async(buf.data_ptr(), 24, sink.data_ptr(), None) == A.CF_ERR_INVALID_ARGUMENT
    assert L.cf_stream_read_async(buf.data_ptr() + 4, 16, sink.data_ptr(), None) == A.CF_ERR_INVALID_ARGUMENT
    assert L.cf_stream_read_async(buf.data_ptr(), 16, None, None) == A.CF_ERR_INVALID_ARGUMENT


def test_cache_and_lds_reads_run(lib):
    import torch
    A = lib
    buf = torch.randint(0, 1 << 30, ((1 << 22) // 4,), dtype=torch.int32, device="cuda:0")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    A.check(A.lib().cf_cache_read_async(buf.data_ptr(), buf.numel() * 4, 2, sink.data_ptr(), None), "cache_read")
    A.check(A.lib().cf_lds_read_async(2, sink.data_ptr(), None), "lds_read")
    torch.cuda.synchronize()
    assert A.lib().cf_cache_read_async(buf.data_ptr(), 16, 0, sink.data_ptr(), None) == A.CF_ERR_INVALID_ARGUMENT
