"""GPU parity of the batched compressed paged-KV decode (cf_kv_paged_attention_batched_async) against the fp64 CPU
oracle evaluated on the oracle-decoded pages. Tolerance (north star): normwise relative error <= 1e-3 with fp32
accumulation, per (sequence, query head) row; f16 operands with hi/lo-split queries keep it near 3e-4 (P in f16)."""
import numpy as np
import pytest

from kv_helpers import head_err, make_seqs, oracle_batched

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _run(dev, codec, seq_tokens, kv_heads, gqa, D, seed, query_pos=None, splits=(0,), shared=None,
         scale_spread=False, raw_groups=None, v_mult=None, cancel=None, page_spread=None):
    import torch
    from chromofold_amd import kv
    data = make_seqs(seq_tokens, kv_heads, D, seed, scale_spread, v_mult, cancel, page_spread)
    tables = None
    if codec == kv.CODEC_RANS_HYBRID:
        parts = []
        for h in range(kv_heads):
            K = data[0][0][h][: (data[0][0].shape[1] // 16) * 16].reshape(-1, 16, D)[:32]
            V = data[0][1][h][: (data[0][1].shape[1] // 16) * 16].reshape(-1, 16, D)[:32]
            parts += [kv.build_table(K), kv.build_table(V)]
        tables = np.concatenate(parts)
    if shared:
        for s, (donor, groups) in shared.items():  # the shared prefix really is the donor's data
            n = groups * 64
            data[s][0][:, :n] = data[donor][0][:, :n]
            data[s][1][:, :n] = data[donor][1][:, :n]
    S = len(seq_tokens)
    kvb = kv.build_batched(codec, lambda s: data[s], S, kv_heads, np.array(seq_tokens), D, tables, dev,
                           keep_host=True, shared=shared, raw_groups=raw_groups)
    rng = np.random.default_rng(seed + 1)
    q = rng.standard_normal((S, kv_heads * gqa, D)).astype(np.float32)
    qp = np.array([t - 1 for t in seq_tokens] if query_pos is None else query_pos, np.uint32)
    sc = 1.0 / np.sqrt(D)
    ref = oracle_batched(kvb, data, q, qp, sc, gqa)
    dq = torch.from_numpy(q).to(dev)
    dqp = torch.from_numpy(qp.view(np.int32)).to(dev)
    for sp in splits:
        out = torch.full_like(dq, float("nan"))
        kvb.attention(dq, out, dqp, sc, splits=sp)
        got = out.cpu().numpy()
        assert np.isfinite(got).all()
        err = head_err(got, ref)
        assert err <= TOL, (codec, sp, err)
    return kvb


@pytest.mark.parametrize("codec", [1, 2])
@pytest.mark.parametrize("D", [128, 64])
def test_batched_ragged(dev, codec, D):
    # ragged lengths: partial last pages, a single-token sequence, lengths not multiples of 64 tokens
    _run(dev, codec, [1, 16, 17, 100, 255, 640, 1029], 2, 4, D, seed=5 + D, splits=(0, 1, 3))


@pytest.mark.parametrize("codec", [1, 2])
def test_batched_causal_query_pos(dev, codec):
    # query positions inside the context: tokens after query_pos are masked
    _run(dev, codec, [300, 300, 64], 3, 4, 128, seed=9, query_pos=[0, 150, 63], splits=(0, 2))


@pytest.mark.parametrize("gqa", [1, 2, 4])
def test_batched_gqa(dev, gqa):
    _run(dev, 2, [200, 333], 2, gqa, 128, seed=13 + gqa)


def test_batched_shared_prefix(dev):
    # sequences 1..3 reuse sequence 0's first 2 page groups = 128 tokens (refcounted prefix blobs)
    _run(dev, 2, [256, 200, 300, 129], 2, 4, 128, seed=21, shared={1: (0, 2), 2: (0, 2), 3: (0, 2)})


@pytest.mark.parametrize("D", [128, 64])
def test_batched_shared_prefix_stored_raw(dev, D):
    # the shared prefix kept as INT8 groups inside the rANS pool (one sequence also has a raw group of its own);
    # the kernel takes each group by its header's codec
    _run(dev, 2, [256, 200, 300, 129], 2, 4, D, seed=23, splits=(0, 2), shared={1: (0, 2), 2: (0, 2), 3: (0, 2)},
         raw_groups={0: 2, 2: 3})


def test_batched_value_spread(dev):
    # outlier channels and tiny / huge tokens: per-page absmax keeps decode exact, output within tolerance
    _run(dev, 2, [512, 96], 2, 4, 128, seed=33, scale_spread=True)


def test_batched_llama_shape_4k(dev):
    """C4 shape at 4k context with 4 sequences (32 q heads, 8 kv heads, hd 128)."""
    _run(dev, 2, [4096] * 4, 8, 4, 128, seed=0xC4, splits=(0,))


# V magnitudes per (sequence, KV head): whole sequences of small or huge V (every page scale small / huge), and one
# sequence whose two heads differ by 1e8. The P.V operand must not lose precision to f16 range: each row is checked
# on its own against the fp64 oracle.
V_MULTS = [[1e-2, 1e-2], [1e-3, 1e-3], [1e-5, 1e-5], [1e7, 1e7], [1e-5, 1e3]]


@pytest.mark.parametrize("codec", [1, 2])
def test_batched_v_magnitudes(dev, codec):
    _run(dev, codec, [4096, 4096, 4100, 4096, 4160], 2, 4, 128, seed=41, splits=(0, 1, 3), v_mult=V_MULTS)


def test_batched_v_magnitudes_hd64(dev):
    _run(dev, 2, [4096, 4096, 4100, 4096, 4160], 2, 4, 64, seed=43, splits=(0, 3), v_mult=V_MULTS)


# Wide workgroups (12 wavefronts, each taking a priority-weighted block of chain pairs, V quads parked in LDS) serve
# launches with at most one (sequence, head) unit per CU whose splits keep >= 24 chain pairs each; splits=1 and 2 on
# these >= 6144-token contexts select them (units x splits <= CUs, 71 and 35 pairs per split), the automatic choice
# (21 splits of 3 pairs) the narrow shape. The pair blocks are static, so the outputs are bitwise reproducible.
@pytest.mark.parametrize("codec", [1, 2])
@pytest.mark.parametrize("D", [128, 64])
def test_batched_wide_workgroups(dev, codec, D):
    _run(dev, codec, [6200, 7000, 6145, 9000, 1, 6400], 2, 4, D, seed=51 + D + codec, splits=(1, 2, 0),
         query_pos=[6199, 3500, 6144, 8999, 0, 100])


def test_batched_wide_raw_and_shared_groups(dev):
    # INT8 groups inside the rANS pool under the wide shape: a shared 4-group prefix (sequences 1, 2 reuse sequence
    # 0's blobs), sequence 3 with 7 leading raw groups (its first coded group, 7, starts its own chain mid-pair)
    _run(dev, 2, [6500, 6300, 7100, 8000], 2, 4, 128, seed=57, splits=(1, 0),
         shared={1: (0, 4), 2: (0, 4)}, raw_groups={0: 4, 3: 7})


def test_batched_wide_v_magnitudes(dev):
    _run(dev, 2, [6144, 6200, 7000, 6150, 6400], 2, 4, 128, seed=59, splits=(1,), v_mult=V_MULTS)


# Cancellation: outputs that are sums of near-opposite page pairs (make_seqs(cancel=1/64)), ~64x smaller than
# sum p |v|. A P.V weight p * v_scale rounded to one f16 (11 significant bits) errs by up to 2^-12 of p v per token,
# independently in the two pages of a pair: about 2e-2 of such an output (a float64 simulation of this data gives
# 1.9e-2 for one f16 and 3.4e-6 for an f16 hi + lo pair). The reference accumulates p v in fp32
# (src/cuda/paged_kv_attention.cu:228-240). Narrow and wide shapes, splits 0/1/2/3, both codecs, head_dim 128 and
# 64, raw and coded groups, every (sequence, query head) row on its own.
@pytest.mark.parametrize("codec", [1, 2])
@pytest.mark.parametrize("D", [128, 64])
def test_batched_cancellation(dev, codec, D):
    _run(dev, codec, [6200, 7000, 6145, 9000, 1, 6400], 2, 4, D, seed=71 + D + codec, splits=(1, 2, 0, 3),
         query_pos=[6199, 3500, 6144, 8999, 0, 100], cancel=1 / 64)


@pytest.mark.parametrize("codec", [1, 2])
def test_batched_page_scale_spread(dev, codec):
    """The pages of one 64-token group share P.V units (the group's largest V scale): V scales spread by up to 2^16
    across the pages of each group (every page of its own magnitude), alone and with cancelling page pairs, through
    the narrow and wide shapes."""
    _run(dev, codec, [6200, 7000, 300, 6400], 2, 4, 128, seed=87 + codec, splits=(1, 0, 3), page_spread=16)
    _run(dev, codec, [6200, 700, 6145], 2, 4, 128, seed=89 + codec, splits=(1, 0), page_spread=12, cancel=1 / 64)


def test_batched_cancellation_short_and_shared(dev):
    _run(dev, 2, [300, 1029, 64, 4096, 700], 3, 4, 128, seed=77, splits=(0, 1, 3), cancel=1 / 64,
         shared={1: (0, 1), 3: (0, 1)}, raw_groups={0: 1, 4: 3})


def test_cascade_cancellation(dev):
    """The cascade's INT8 prefix pass and the batched suffix pass over near-cancelling pairs."""
    tokens = [4096, 4160, 1100, 4200, 700]
    kvb, data, q, qp, sc, got = _cascade_case(dev, 4, tokens, 10, seed=101, cancel=1 / 64)
    assert np.isfinite(got).all()
    ref = oracle_batched(kvb, data, q, qp, sc, 4)
    assert head_err(got, ref) <= TOL


def test_batched_rejects_bad_desc(dev):
    import ctypes as C
    import torch
    from chromofold_amd import _abi as A
    from chromofold_amd import kv
    kvb = _run(dev, 1, [32], 1, 4, 128, seed=1)
    q = torch.zeros((1, 4, 128), device=dev)
    o = torch.zeros_like(q)
    qp = torch.zeros(1, dtype=torch.int32, device=dev)
    d = kvb.desc(q, o, qp, 0.1)
    L = A.lib()
    for field, val, st in [("struct_size", 8, 1), ("abi_version", 99, 1), ("codec", 7, 2), ("head_dim", 96, 2),
                           ("query_head_count", 5, 2), ("queries", None, 1)]:
        bad = kv.cf_kv_batched_desc.from_buffer_copy(d)
        setattr(bad, field, val)
        assert L.cf_kv_paged_attention_batched_async(C.byref(bad), None) == st, field


def test_batched_full_c4_32k_every_sequence_torch_reference(dev):
    """The benchmark's full paged-KV shape — 32 sequences x 32768 tokens, 8 KV / 32 q heads, hd 128 — sealed on the device,
    then EVERY output row against an independent float64 torch reference over the dequantised values (quantised
    here with torch: per-page absmax / 127, IEEE division, round half to even). Covers every group of every
    (sequence, head) at the benchmark's real size. Bar: max abs error <= 1e-3 x max |ref| per (sequence, query head)
    row."""
    import torch
    from chromofold_amd import kv
    S, T, H, QH, D = 32, 32768, 8, 32, 128
    gqa = QH // H
    gen = torch.Generator(device=dev)
    gen.manual_seed(0xC4)
    K = torch.randn((S, H, T, D), generator=gen, device=dev)
    V = torch.randn((S, H, T, D), generator=gen, device=dev)
    Kh = K[0, 0, :512].cpu().numpy().reshape(-1, 16, D)
    Vh = V[0, 0, :512].cpu().numpy().reshape(-1, 16, D)
    tables = torch.from_numpy(np.concatenate([t for _ in range(H) for t in (kv.build_table(Kh), kv.build_table(Vh))]))
    kvb = kv.seal_device(kv.CODEC_RANS_HYBRID, K, V, tables.to(dev))
    q = torch.randn((S, QH, D), generator=gen, device=dev)
    qp = torch.full((S,), T - 1, dtype=torch.int32, device=dev)
    out = torch.full_like(q, float("nan"))
    sc = 1.0 / np.sqrt(D)
    kvb.attention(q, out, qp, sc)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()

    def deq(x):  # [T, D] -> dequantised float64
        p = x.view(-1, 16, D)
        m = p.abs().amax(dim=(1, 2), keepdim=True)
        s = torch.where(m == 0, torch.ones_like(m), m / 127.0)
        return (torch.clamp(torch.round(p / s), -128, 127) * s).view(T, D).double()

    worst = 0.0
    for s in range(S):
        ref = torch.empty((QH, D), dtype=torch.float64, device=dev)
        for h in range(H):
            kd, vd = deq(K[s, h]), deq(V[s, h])
            qs = q[s, h * gqa:(h + 1) * gqa].double()
            p = torch.softmax((qs @ kd.T) * sc, dim=-1)
            ref[h * gqa:(h + 1) * gqa] = p @ vd
        err = float(((out[s].double() - ref).abs().amax(dim=1) / ref.abs().amax(dim=1)).max())
        worst = max(worst, err)
        assert err <= 1e-3, (s, err)
    print(f"full C4 32k: worst normwise error over 32 x 32 (sequence, head) rows {worst:.3e}")


def _cascade_case(dev, gqa, seq_tokens, shared, seed, query_pos=None, raw_prefix=True, D=128, kv_heads=2,
                  v_mult=None, splits=0, cancel=None):
    import torch
    from chromofold_amd import kv
    data = make_seqs(seq_tokens, kv_heads, D, seed, v_mult=v_mult, cancel=cancel)
    n = shared * 64
    for s in range(1, len(seq_tokens)):  # every sequence starts with sequence 0's prefix
        data[s][0][:, :n] = data[0][0][:, :n]
        data[s][1][:, :n] = data[0][1][:, :n]
    parts = []
    for h in range(kv_heads):
        parts += [kv.build_table(data[0][0][h][:512].reshape(-1, 16, D)), kv.build_table(data[0][1][h][:512].reshape(-1, 16, D))]
    tables = np.concatenate(parts)
    S = len(seq_tokens)
    kvb = kv.build_batched(kv.CODEC_RANS_HYBRID, lambda s: data[s], S, kv_heads, np.array(seq_tokens), D, tables, dev,
                           keep_host=True, shared={s: (0, shared) for s in range(1, S)},
                           raw_groups={0: shared} if raw_prefix else None)
    rng = np.random.default_rng(seed + 1)
    q = rng.standard_normal((S, kv_heads * gqa, D)).astype(np.float32)
    qp = np.array([t - 1 for t in seq_tokens] if query_pos is None else query_pos, np.uint32)
    sc = 1.0 / np.sqrt(D)
    dq = torch.from_numpy(q).to(dev)
    dqp = torch.from_numpy(qp.view(np.int32)).to(dev)
    out = torch.full_like(dq, float("nan"))
    kvb.attention(dq, out, dqp, sc, splits=splits, shared_groups=shared)
    return kvb, data, q, qp, sc, out.cpu().numpy()


@pytest.mark.parametrize("gqa,seq_tokens,query_pos", [
    (4, [512, 300, 129, 700, 200] + [260] * 14, None),         # 19 sequences: a partly filled 16-sequence tile
    (2, [256, 200, 300, 129], [255, 150, 120, 128]),           # GQA 2; one query sees only part of the prefix
    (1, [1024] * 3 + [640], None),                              # long prefix split over several workgroups
])
def test_cascade_shared_prefix_vs_oracle(dev, gqa, seq_tokens, query_pos):
    """cf_kv_paged_attention_cascade_async: the INT8 prefix shared by every sequence is streamed once per KV head
    for all of them, each sequence's own rANS groups by the batched kernel, the partials merged. Against the fp64
    oracle over the oracle-decoded pages (same bar as the batched tests)."""
    shared = 2 if min(seq_tokens) < 1024 else 10
    kvb, data, q, qp, sc, got = _cascade_case(dev, gqa, seq_tokens, shared, seed=61 + gqa, query_pos=query_pos)
    assert np.isfinite(got).all()
    ref = oracle_batched(kvb, data, q, qp, sc, gqa)
    assert head_err(got, ref) <= TOL


@pytest.mark.parametrize("query_pos", [None, [255, 100, 50]])
def test_cascade_rejects_a_coded_prefix_loudly(dev, query_pos):
    # the prefix pass reads INT8 groups only: a rANS-coded prefix turns every output into NaN instead of a wrong
    # value, also for queries that see nothing but prefix tokens (positions 100 and 50 < the 128-token prefix)
    _, _, _, _, _, got = _cascade_case(dev, 4, [256, 300, 200], 2, seed=71, raw_prefix=False, query_pos=query_pos)
    assert np.isnan(got).all()


def test_cascade_argument_checks(dev):
    import ctypes as C
    import torch
    from chromofold_amd import _abi as A
    from chromofold_amd import kv
    kvb, *_ = _cascade_case(dev, 4, [256, 200], 2, seed=81)
    q = torch.zeros((2, 8, 128), device=dev)
    o = torch.zeros_like(q)
    qp = torch.zeros(2, dtype=torch.int32, device=dev)
    d = kvb.desc(q, o, qp, 0.1, shared_groups=2)
    L = A.lib()
    assert L.cf_kv_paged_attention_cascade_async(C.byref(d), 0, None) == A.CF_ERR_INVALID_ARGUMENT
    assert L.cf_kv_paged_attention_cascade_async(C.byref(d), kvb.max_groups + 1, None) == A.CF_ERR_INVALID_ARGUMENT
    small = kv.cf_kv_batched_desc.from_buffer_copy(d)
    small.workspace_bytes = 16
    assert L.cf_kv_paged_attention_cascade_async(C.byref(small), 2, None) == A.CF_ERR_INVALID_ARGUMENT
    assert L.cf_kv_cascade_workspace_bytes(C.byref(d), 0) == 0


@pytest.mark.parametrize("seed", [5, 6])
def test_cascade_random_suffixes(dev, seed):
    """Random sequence count (17..40), random own lengths after a 3-group shared prefix, random query positions
    (some inside the prefix, some at the end), GQA 4."""
    rng = np.random.default_rng(seed)
    S = int(rng.integers(17, 41))
    shared = 3
    tokens = [192 + int(rng.integers(0, 700)) for _ in range(S)]
    qpos = [int(rng.integers(100, t)) if rng.random() < 0.3 else t - 1 for t in tokens]
    kvb, data, q, qp, sc, got = _cascade_case(dev, 4, tokens, shared, seed=90 + seed, query_pos=qpos)
    assert np.isfinite(got).all()
    ref = oracle_batched(kvb, data, q, qp, sc, 4)
    assert head_err(got, ref) <= TOL


def test_cascade_wide_suffix_after_odd_prefix(dev):
    """A 3-group (odd) INT8 prefix, then long own suffixes decoded by wide workgroups (splits=1: 110 suffix groups):
    the suffix launch starts at group 3, in the middle of chain pair (2, 3)."""
    tokens = [192 + 6400, 192 + 7000, 192 + 6200]
    kvb, data, q, qp, sc, got = _cascade_case(dev, 4, tokens, 3, seed=63, splits=1,
                                              query_pos=[192 + 6399, 150, 192 + 3000])
    assert np.isfinite(got).all()
    ref = oracle_batched(kvb, data, q, qp, sc, 4)
    assert head_err(got, ref) <= TOL


@pytest.mark.parametrize("v_mult", [[[1e-5, 1e-5]] * 4, [[1e7, 1e7]] * 4,
                                    [[1e-3, 1e-3], [1e-5, 1e-5], [1e7, 1e7], [1e-2, 1.0]]])
def test_cascade_v_magnitudes(dev, v_mult):
    """Cascade decode with small / huge V: a 40-group (2560-token) INT8 prefix shared by every sequence (of sequence
    0's magnitude) and each sequence's own rANS groups (of its own magnitude), >= 4096 tokens each."""
    tokens = [4096, 4160, 4096, 4200]
    kvb, data, q, qp, sc, got = _cascade_case(dev, 4, tokens, 40, seed=97, v_mult=v_mult)
    assert np.isfinite(got).all()
    ref = oracle_batched(kvb, data, q, qp, sc, 4)
    assert head_err(got, ref) <= TOL


def test_c5_long_context_131k_every_row(dev):
    """BASELINE C5's long-context shape: 4 sequences x 131072 tokens, 8 KV / 32 q heads, hd 128, sealed on the
    device (2048 groups per sequence and head), one decode token each. Every (sequence, query head) row against the
    float64 oracle decoding the pool's own blobs (O.kv_pool_attention, all host threads), normwise <= 1e-3."""
    import torch
    import oracle as O
    from chromofold_amd import kv
    S, T, H, QH, D = 4, 131072, 8, 32, 128
    gen = torch.Generator(device=dev)
    gen.manual_seed(0xC5)
    K = torch.randn((S, H, T, D), generator=gen, device=dev)
    V = torch.randn((S, H, T, D), generator=gen, device=dev)
    Kh = K[0, 0, :512].cpu().numpy().reshape(-1, 16, D)
    Vh = V[0, 0, :512].cpu().numpy().reshape(-1, 16, D)
    tables = np.concatenate([t for _ in range(H) for t in (kv.build_table(Kh), kv.build_table(Vh))])
    kvb = kv.seal_device(kv.CODEC_RANS_HYBRID, K, V, torch.from_numpy(tables).to(dev))
    del K, V
    q = torch.randn((S, QH, D), generator=gen, device=dev)
    qp = torch.tensor([T - 1, T - 1, 70000, 131000], dtype=torch.int32, device=dev)
    out = torch.full_like(q, float("nan"))
    sc = 1.0 / np.sqrt(D)
    kvb.attention(q, out, qp, sc)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    ref = O.kv_pool_attention(kvb.pool.cpu().numpy(), kvb.group_offsets.cpu().numpy().view(np.uint32),
                              np.full(S, T, np.uint32), qp.cpu().numpy().view(np.uint32), tables, q.cpu().numpy(),
                              H, D, sc)
    err = np.abs(got - ref).max(axis=2) / np.abs(ref).max(axis=2)
    assert err.max() <= TOL, err.max()
    print(f"C5 4 x 131072: worst normwise error over {err.size} rows {err.max():.3e}")


def test_c5_shared_prefix_full_shape_every_row(dev):
    """BASELINE C5's shared-prefix shape at full size: 256 sequences x (8192 shared + 512 own) tokens, 8 KV / 32 q
    heads, hd 128. The prefix is stored once, as INT8 groups inside the rANS pool, and referenced from every
    sequence's group table; each sequence's own 512 tokens are rANS-coded. The cascade entry point (the prefix
    streamed once per KV head for all 256 query sets) and the batched entry point on the same pool; query positions
    at the end, inside the own tokens and inside the prefix. Every (sequence, query head) row against the float64
    oracle decoding the pool's own blobs (O.kv_pool_attention), normwise <= 1e-3."""
    import torch
    import oracle as O
    from chromofold_amd import kv
    S, P, U, H, QH, D = 256, 8192, 512, 8, 32, 128
    T, pg = P + U, P // 64
    rng = np.random.default_rng(0xC5A)
    prefix = (rng.standard_normal((H, P, D), dtype=np.float32), rng.standard_normal((H, P, D), dtype=np.float32))
    seeds = rng.integers(0, 2 ** 63, size=S)

    def src(s):
        g = np.random.default_rng(int(seeds[s]))
        Ks = np.zeros((H, T, D), np.float32)
        Vs = np.zeros((H, T, D), np.float32)
        if s == 0:
            Ks[:, :P], Vs[:, :P] = prefix
        Ks[:, P:] = g.standard_normal((H, U, D), dtype=np.float32)
        Vs[:, P:] = g.standard_normal((H, U, D), dtype=np.float32)
        return Ks, Vs

    tables = np.concatenate([t for h in range(H) for t in (kv.build_table(prefix[0][h, :512].reshape(-1, 16, D)),
                                                           kv.build_table(prefix[1][h, :512].reshape(-1, 16, D)))])
    kvb = kv.build_batched(kv.CODEC_RANS_HYBRID, src, S, H, np.full(S, T, np.uint32), D, tables, dev,
                           shared={s: (0, pg) for s in range(1, S)}, raw_groups={0: pg})
    q = rng.standard_normal((S, QH, D), dtype=np.float32)
    qp = np.full(S, T - 1, np.uint32)
    qp[1::7] = rng.integers(P, T - 1, size=qp[1::7].size)  # inside the own tokens
    qp[3::11] = rng.integers(0, P, size=qp[3::11].size)    # inside the shared prefix
    dq = torch.from_numpy(q).to(dev)
    dqp = torch.from_numpy(qp.view(np.int32)).to(dev)
    sc = 1.0 / np.sqrt(D)
    ref = O.kv_pool_attention(kvb.pool.cpu().numpy(), kvb.group_offsets.cpu().numpy().view(np.uint32),
                              np.full(S, T, np.uint32), qp, tables, q, H, D, sc)
    for shared_groups in (pg, 0):  # cascade, then batched
        out = torch.full_like(dq, float("nan"))
        kvb.attention(dq, out, dqp, sc, shared_groups=shared_groups)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert np.isfinite(got).all(), shared_groups
        err = np.abs(got - ref).max(axis=2) / np.abs(ref).max(axis=2)
        assert err.max() <= TOL, (shared_groups, err.max())
        print(f"C5 256 x (8192 + 512), shared_groups={shared_groups}: worst normwise error {err.max():.3e}")


def test_c4_4k_batch_32_every_row(dev):
    """BASELINE C4 at its 4k context: 32 sequences x 4096 tokens, 8 KV / 32 q heads, hd 128, sealed on the device,
    run with the automatic launch plan (the narrow shape with context splits and the merge kernel). Every
    (sequence, query head) row against the float64 oracle decoding the pool's own blobs, normwise <= 1e-3."""
    import torch
    import oracle as O
    from chromofold_amd import kv
    S, T, H, QH, D = 32, 4096, 8, 32, 128
    gen = torch.Generator(device=dev)
    gen.manual_seed(0xC44)
    K = torch.randn((S, H, T, D), generator=gen, device=dev)
    V = torch.randn((S, H, T, D), generator=gen, device=dev)
    tables = np.concatenate([t for _ in range(H) for t in (kv.build_table(K[0, 0, :512].cpu().numpy().reshape(-1, 16, D)),
                                                           kv.build_table(V[0, 0, :512].cpu().numpy().reshape(-1, 16, D)))])
    kvb = kv.seal_device(kv.CODEC_RANS_HYBRID, K, V, torch.from_numpy(tables).to(dev))
    del K, V
    q = torch.randn((S, QH, D), generator=gen, device=dev)
    qp = torch.full((S,), T - 1, dtype=torch.int32, device=dev)
    qp[5], qp[17] = 2000, 63
    out = torch.full_like(q, float("nan"))
    sc = 1.0 / np.sqrt(D)
    kvb.attention(q, out, qp, sc)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    ref = O.kv_pool_attention(kvb.pool.cpu().numpy(), kvb.group_offsets.cpu().numpy().view(np.uint32),
                              np.full(S, T, np.uint32), qp.cpu().numpy().view(np.uint32), tables, q.cpu().numpy(),
                              H, D, sc)
    err = np.abs(got - ref).max(axis=2) / np.abs(ref).max(axis=2)
    assert err.max() <= TOL, err.max()
    print(f"C4 32 x 4096: worst normwise error over {err.size} rows {err.max():.3e}")
