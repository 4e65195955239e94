"""GPU index construction (cf_rrrw_build / cf_rrrw_build_copy, cf_suffix_array + cf_fm_build_aux) against the
oracle builder, which is itself pinned byte for byte to the reference's tools/build_index (and to tiny.cfrw /
tiny.cffm): every array identical, then queries on the GPU-built index against closed forms."""
import numpy as np
import pytest

import cf_fixtures as F
import oracle as O

pytestmark = pytest.mark.gpu

FIELDS = ["classes", "offsets", "rank_a", "rank_d", "off_a", "off_d", "offbase", "zeros"]


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _host(t, dtype):
    return t.cpu().numpy().view(dtype)


def _check_rrrw(idx, lay, ref):
    dt = {"classes": np.uint32, "offsets": np.uint32, "rank_a": np.int32, "rank_d": np.uint16, "off_a": np.int32,
          "off_d": np.uint16, "offbase": np.int32, "zeros": np.int32}
    for f in FIELDS:
        got = _host(idx.tensors[f], dt[f])
        assert np.array_equal(got, getattr(ref, f)), f
    assert (idx.cwords, idx.nsb, idx.na) == (ref.cwords, ref.nsb, ref.na)
    assert lay.rrr_bytes == ref.rrr_bytes


@pytest.mark.parametrize("n,bits,seed", [(1, 1, 0), (15, 3, 1), (256, 4, 2), (4097, 7, 3), (65536, 15, 4),
                                         (100003, 9, 5), (30000, 16, 6), (960 * 64 + 7, 2, 7)])
def test_rrrw_build_matches_oracle(dev, n, bits, seed):
    import torch
    from chromofold_amd.search import build_rrrw
    rng = np.random.default_rng(seed)
    ranks = np.arange(1, (1 << bits) + 1, dtype=np.float64)
    p = ranks ** -1.1
    tok = rng.choice(1 << bits, size=n, p=p / p.sum()).astype(np.uint32)
    idx, lay = build_rrrw(torch.from_numpy(tok.view(np.int32)).to(dev), bits)
    _check_rrrw(idx, lay, O.rrrw_build(tok, bits))
    pos = rng.integers(0, n, 2000).astype(np.uint32)
    from chromofold_amd.search import to_u32, u32_dev
    assert np.array_equal(to_u32(idx.access(u32_dev(pos, dev))), tok[pos])


def test_rrrw_build_tiny_cfrw(dev):
    """Rebuild the committed fixture from its decoded BWT: every array equals the file."""
    import torch
    from chromofold_amd.search import build_rrrw
    d = F.load_cfrw()
    w = O.RrrwArrays(d["bits"], d["cwords"], d["nsb"], d["na"], *[d[f] for f in FIELDS])
    bwt = O.rrrw_access(w, np.arange(d["n"], dtype=np.uint32))
    idx, lay = build_rrrw(torch.from_numpy(bwt.view(np.int32)).to(dev), d["bits"])
    for f, dt in zip(FIELDS, [np.uint32, np.uint32, np.int32, np.uint16, np.int32, np.uint16, np.int32, np.int32]):
        assert np.array_equal(_host(idx.tensors[f], dt), d[f]), f
    assert lay.rrr_bytes == d["rrr_bytes"]


@pytest.mark.parametrize("n,V,sample,seed", [(8192, 64, 16, 1), (50000, 3000, 32, 2), (1, 5, 4, 3), (777, 2, 1, 4)])
def test_fm_build_matches_oracle(dev, n, V, sample, seed):
    import torch
    from chromofold_amd.search import build_fm
    rng = np.random.default_rng(seed)
    ranks = np.arange(1, V + 1, dtype=np.float64)
    p = ranks ** -1.1
    tok = rng.choice(V, size=n, p=p / p.sum()).astype(np.int32)
    fm, info = build_fm(torch.from_numpy(tok).to(dev), sample)
    ref, bwt = O.fm_build(tok.astype(np.uint32), sample)
    assert np.array_equal(info["bwt"].cpu().numpy(), bwt)
    for f in ("C", "mwords", "msb", "sval"):
        assert np.array_equal(fm.tensors[f].cpu().numpy().view(getattr(ref, f).dtype), getattr(ref, f)), f
    _check_rrrw(fm.w, info["layout"], ref.w)
    # queries on the GPU-built index: count of substrings cut from the text equals naive search
    s = O.fm_text(tok.astype(np.uint32))
    L = min(6, n)
    starts = rng.integers(0, n - L + 1, 64)
    pats = [s[a:a + L] for a in starts]
    pat = np.concatenate(pats).astype(np.int32)
    pstart = (np.arange(64) * L).astype(np.int32)
    plen = np.full(64, L, np.int32)
    cnt = fm.count(torch.from_numpy(pat).to(dev), torch.from_numpy(pstart).to(dev), torch.from_numpy(plen).to(dev))
    exp = np.array([O.naive_count(s, q) for q in pats], np.int32)
    assert np.array_equal(cnt.cpu().numpy(), exp)


def _inverse_bwt(bwt: np.ndarray, C: np.ndarray) -> np.ndarray:
    """Text s (ending in the sentinel 0) from its BWT by LF steps from row 0 (the sentinel's suffix)."""
    n = bwt.size
    occ = np.zeros(n, np.int64)
    seen = np.zeros(C.size, np.int64)
    for i, c in enumerate(bwt):
        occ[i] = seen[c]
        seen[c] += 1
    s = np.zeros(n, np.int32)
    row = 0
    for k in range(n - 2, -1, -1):
        c = bwt[row]
        s[k] = c
        row = C[c] + occ[row]
    return s


def test_gpu_built_files_equal_reference_fixtures(dev, tmp_path):
    """The on-disk builder path: build on the GPU, write .cfrw / .cffm with the library's writer, and get the
    reference's committed files back byte for byte (h0 included; packed_bytes aside, see below)."""
    import torch
    from chromofold_amd import search as S
    d = F.load_cfrw()
    w = O.RrrwArrays(d["bits"], d["cwords"], d["nsb"], d["na"], *[d[f] for f in FIELDS])
    bwt = O.rrrw_access(w, np.arange(d["n"], dtype=np.uint32))
    sym = torch.from_numpy(bwt.view(np.int32)).to(dev)
    idx, lay = S.build_rrrw(sym, d["bits"])
    out = str(tmp_path / "gpu.cfrw")
    S.save_cfrw(out, idx, lay, d["vocab"], sym, {k: d[k] for k in ("pos", "access_golden", "rank_c", "rank_i",
                                                                   "rank_golden")})
    got, ref = open(out, "rb").read(), open(F._path("tiny.cfrw"), "rb").read()
    # packed_bytes (file offset 60..68) is the packed wavelet's footprint figure; tiny.cfrw took it from the Python
    # exporter's warp_compress package, the library uses the C++ builder's formula (pinned in test_index_io.py)
    assert got[:60] + got[68:] == ref[:60] + ref[68:]

    f = F.load_cffm()
    wf = O.RrrwArrays(f["bits"], f["cwords"], f["nsb"], f["na"], *[f[k] for k in FIELDS])
    fbwt = O.rrrw_access(wf, np.arange(f["n"], dtype=np.uint32)).astype(np.int64)
    s = _inverse_bwt(fbwt, f["C"].astype(np.int64))
    assert s[-1] == 0 and (s[:-1] > 0).all()
    tokens = torch.from_numpy((s[:-1] - 1).astype(np.int32)).to(dev)
    fm, info = S.build_fm(tokens, f["sa_sample"])
    out = str(tmp_path / "gpu.cffm")
    S.save_cffm(out, fm, info["layout"], f["vocab"], {k: f[k] for k in ("pat", "pstart", "plen", "count_golden",
                                                                         "locoff", "locpos")})
    assert open(out, "rb").read() == open(F._path("tiny.cffm"), "rb").read()
