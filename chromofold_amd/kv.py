"""Host-side mirror of the compressed paged-KV interface.

Two entry points are mirrored:
  * the batched multi-sequence decode of include/chromofold/kv_codec_ext.h (INT8 / RANS_HYBRID page blobs in one
    device pool, per-(sequence, head) page tables, split-context workspace) — the benchmark path;
  * the legacy single-sequence seam cf_kv_paged_attention_async of include/chromofold/kv_cuda.h (see legacy.py).

Encoding happens either on the host through the library's C encoder (cf_kv_encode_groups) or on the device
(cf_kv_encode_groups_async, the same bytes); pools, page tables, queries and outputs live in HBM as torch tensors.
Every launch goes through libchromofold.so.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _abi as A

CODEC_INT8, CODEC_RANS_HYBRID = 1, 2
PAGE_TOKENS = 16
TABLE_BYTES = 16384
EXT_ABI_VERSION = 4
GROUP_PAGES = 4
GROUP_TOKENS = PAGE_TOKENS * GROUP_PAGES


class cf_kv_batched_desc(C.Structure):
    _fields_ = [("struct_size", A.U32), ("abi_version", A.U32), ("codec", A.U32), ("seq_count", A.U32),
                ("kv_head_count", A.U32), ("query_head_count", A.U32), ("head_dim", A.U32), ("max_groups", A.U32),
                ("pool", A.P), ("group_offsets", A.P), ("seq_tokens", A.P), ("query_pos", A.P), ("tables", A.P),
                ("queries", A.P), ("output", A.P), ("softmax_scale", A.F32), ("splits", A.U32),
                ("workspace", A.P), ("workspace_bytes", A.U64)]


A.declare("cf_kv_encode_groups", A.I32, [A.U32, A.P, A.P, A.U64, A.P, A.P, A.P, A.U32, A.P, A.P, A.P, A.P, A.U64,
                                         A.U64, A.P, A.P, A.U32])
A.declare("cf_kv_encode_group", A.I32, [A.U32, A.P, A.P, A.U32, A.P, A.U32, A.P, A.P, A.U32, A.U32, A.P, A.U64, A.P])
A.declare("cf_kv_rans_build_table", A.I32, [A.P, A.P])
A.declare("cf_kv_rans_page_histogram", A.I32, [A.P, A.U32, A.U32, A.P])
A.declare("cf_kv_group_blob_max_bytes", A.U64, [A.U32, A.U32])
A.declare("cf_kv_batched_workspace_bytes", A.U64, [A.P])
A.declare("cf_kv_validate_batched_desc", A.I32, [A.P])
A.declare("cf_kv_paged_attention_batched_async", A.I32, [A.P, A.P])
A.declare("cf_kv_cascade_workspace_bytes", A.U64, [A.P, A.U32])
A.declare("cf_kv_paged_attention_cascade_async", A.I32, [A.P, A.U32, A.P])
A.declare("cf_kv_encode_groups_workspace_bytes", A.U64, [A.U32, A.U32, A.U64, A.U32])
A.declare("cf_kv_encode_groups_async", A.I32, [A.U32, A.P, A.P, A.U64, A.P, A.P, A.P, A.U32, A.P, A.U32, A.P, A.P,
                                               A.P, A.U64, A.U64, A.P, A.P, A.P, A.P, A.U64, A.P])


def _np_ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def pair_flags(group_index: np.ndarray, first_coded: int = 0) -> np.ndarray:
    """`continues` flags for groups listed in token order with absolute group indices `group_index` (one sequence and
    head): an odd group continues the chain of the even group before it when that group is in the list and coded
    (index >= first_coded)."""
    g = np.asarray(group_index, np.int64)
    return ((g % 2 == 1) & (g - 1 >= max(first_coded, int(g.min()) if g.size else 0))).astype(np.uint8)


def build_table(pages: np.ndarray) -> np.ndarray:
    """Table blob from the joint big-bit histogram of sample pages [n, tokens<=16, D] (fp32)."""
    L = A.lib()
    pages = np.ascontiguousarray(pages, np.float32)
    hist = np.zeros(256, np.uint64)
    for p in pages:
        A.check(L.cf_kv_rans_page_histogram(_np_ptr(p), p.shape[0], p.shape[1], _np_ptr(hist)), "histogram")
    out = np.zeros(TABLE_BYTES, np.uint8)
    A.check(L.cf_kv_rans_build_table(_np_ptr(hist), _np_ptr(out)), "build_table")
    return out


def encode_groups(codec: int, keys: np.ndarray, values: np.ndarray, head_dim: int, tables: np.ndarray | None,
                  first_page: np.ndarray, page_counts: np.ndarray, heads: np.ndarray | None = None,
                  token_counts: np.ndarray | None = None, threads: int = 0,
                  continues: np.ndarray | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Encode page groups of page-major pages keys/values [n_pages, 16, D] -> (blob bytes, offsets/16).
    continues[i] = 1 codes group i as the second group of group i - 1's chain pair (see pair_flags)."""
    L = A.lib()
    keys = np.ascontiguousarray(keys, np.float32)
    values = np.ascontiguousarray(values, np.float32)
    first_page = np.ascontiguousarray(first_page, np.uint64)
    page_counts = np.ascontiguousarray(page_counts, np.uint32)
    n = first_page.size
    cap = int(L.cf_kv_group_blob_max_bytes(codec, head_dim)) * n
    pool = np.zeros(cap, np.uint8)
    offs = np.zeros(n, np.uint32)
    end = C.c_uint64(0)
    hd = None if heads is None else np.ascontiguousarray(heads, np.uint32)
    tc = None if token_counts is None else np.ascontiguousarray(token_counts, np.uint32)
    ct = None if continues is None else np.ascontiguousarray(continues, np.uint8)
    st = L.cf_kv_encode_groups(codec, _np_ptr(keys), _np_ptr(values), n, _np_ptr(first_page), _np_ptr(page_counts),
                               _np_ptr(tc), head_dim, _np_ptr(tables), _np_ptr(hd), _np_ptr(ct), _np_ptr(pool), cap,
                               0, _np_ptr(offs), C.byref(end), threads)
    A.check(st, "cf_kv_encode_groups")
    return pool[:end.value], offs


def _dptr(t):
    return None if t is None else t.data_ptr()


@dataclass
class DeviceEncodeResult:
    offsets: torch.Tensor    # [ngroups] int32 view of the u32 pool offsets / 16
    pool_end: torch.Tensor   # [1] int64 (u64 first free byte)
    status: torch.Tensor     # [1] int32 (cf_status of the device-side outcome)


def encode_groups_device(codec: int, keys: torch.Tensor, values: torch.Tensor, head_dim: int,
                         tables: torch.Tensor | None, first_page: torch.Tensor, page_counts: torch.Tensor,
                         pool: torch.Tensor, pool_at: int = 0, heads: torch.Tensor | None = None,
                         token_counts: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                         stream=None, continues: torch.Tensor | None = None) -> DeviceEncodeResult:
    """cf_kv_encode_groups_async on device tensors: keys/values fp32 [n_pages, 16, D], first_page int64,
    page_counts/heads/token_counts int32 (u32 bit patterns), continues uint8 (see pair_flags), tables uint8 (table
    blobs), pool uint8. Asynchronous: read `status` after the stream has run. The workspace is allocated here when
    not given (the C entry point itself allocates nothing)."""
    L = A.lib()
    n = first_page.numel()
    tcount = 0 if tables is None else tables.numel() // TABLE_BYTES
    ws_bytes = int(L.cf_kv_encode_groups_workspace_bytes(codec, head_dim, n, tcount))
    if ws_bytes == 0:
        raise A.CfError(A.CF_ERR_INVALID_ARGUMENT, "cf_kv_encode_groups_workspace_bytes")
    if workspace is None or workspace.numel() < ws_bytes:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=pool.device)
    offs = torch.empty(n, dtype=torch.int32, device=pool.device)
    end = torch.zeros(1, dtype=torch.int64, device=pool.device)
    status = torch.full((1,), -1, dtype=torch.int32, device=pool.device)
    s = (stream if stream is not None else torch.cuda.current_stream()).cuda_stream
    st = L.cf_kv_encode_groups_async(codec, keys.data_ptr(), values.data_ptr(), n, first_page.data_ptr(),
                                     page_counts.data_ptr(), _dptr(token_counts), head_dim, _dptr(tables), tcount,
                                     _dptr(heads), _dptr(continues), pool.data_ptr(), pool.numel(), pool_at,
                                     offs.data_ptr(),
                                     end.data_ptr(), status.data_ptr(), workspace.data_ptr(), workspace.numel(), s)
    A.check(st, "cf_kv_encode_groups_async")
    return DeviceEncodeResult(offs, end, status)


@dataclass
class BatchedKv:
    """Device-resident pages of `seq_count` sequences x `kv_heads` heads for the batched decode entry point."""
    codec: int
    seq_count: int
    kv_heads: int
    head_dim: int
    max_groups: int
    pool: torch.Tensor                 # uint8 [bytes]
    group_offsets: torch.Tensor        # int32 [S, H, max_groups] (u32 bits)
    seq_tokens: torch.Tensor           # int32 [S]
    tables: torch.Tensor | None        # uint8 [2H * 16 KiB]
    host_pool: np.ndarray | None = None
    host_offsets: np.ndarray | None = None
    host_tables: np.ndarray | None = None
    workspace: torch.Tensor | None = None
    stats: dict = field(default_factory=dict)

    @property
    def pool_bytes(self) -> int:
        return int(self.pool.numel())

    def desc(self, queries: torch.Tensor, output: torch.Tensor, query_pos: torch.Tensor, softmax_scale: float,
             splits: int = 0, shared_groups: int = 0) -> cf_kv_batched_desc:
        """Descriptor (with a workspace of this object's) for attention(); shared_groups > 0 sizes the workspace
        for the cascade entry point."""
        d = cf_kv_batched_desc()
        d.struct_size = C.sizeof(cf_kv_batched_desc)
        d.abi_version = EXT_ABI_VERSION
        d.codec = self.codec
        d.seq_count = self.seq_count
        d.kv_head_count = self.kv_heads
        d.query_head_count = queries.shape[1]
        d.head_dim = self.head_dim
        d.max_groups = self.max_groups
        d.pool = self.pool.data_ptr()
        d.group_offsets = self.group_offsets.data_ptr()
        d.seq_tokens = self.seq_tokens.data_ptr()
        d.query_pos = query_pos.data_ptr()
        d.tables = None if self.tables is None else self.tables.data_ptr()
        d.queries = queries.data_ptr()
        d.output = output.data_ptr()
        d.softmax_scale = softmax_scale
        d.splits = splits
        if shared_groups:
            need = int(A.lib().cf_kv_cascade_workspace_bytes(C.byref(d), shared_groups))
            if need == 0:
                raise ValueError("cascade decode needs head_dim 128 and 1 <= shared_groups <= max_groups")
        else:
            need = int(A.lib().cf_kv_batched_workspace_bytes(C.byref(d)))
        if need:
            if self.workspace is None or self.workspace.numel() < need:
                self.workspace = torch.empty(need, dtype=torch.uint8, device=self.pool.device)
            d.workspace = self.workspace.data_ptr()
            d.workspace_bytes = self.workspace.numel()
        return d

    def attention(self, queries: torch.Tensor, output: torch.Tensor, query_pos: torch.Tensor,
                  softmax_scale: float, splits: int = 0, stream=None, desc: cf_kv_batched_desc | None = None,
                  shared_groups: int = 0):
        """Batched decode; shared_groups > 0 uses the cascade entry point (the first shared_groups groups of every
        sequence are sequence 0's, stored as INT8 blobs), with a descriptor made by desc(..., shared_groups=)."""
        d = desc if desc is not None else self.desc(queries, output, query_pos, softmax_scale, splits, shared_groups)
        s = (stream if stream is not None else torch.cuda.current_stream()).cuda_stream
        if shared_groups:
            A.check(A.lib().cf_kv_paged_attention_cascade_async(C.byref(d), shared_groups, s),
                    "cf_kv_paged_attention_cascade_async")
        else:
            A.check(A.lib().cf_kv_paged_attention_batched_async(C.byref(d), s), "cf_kv_paged_attention_batched_async")


def seal_device(codec: int, keys: torch.Tensor, values: torch.Tensor, tables: torch.Tensor | None,
                stream=None) -> BatchedKv:
    """Seal dense device K/V [seq_count, kv_heads, T, D] fp32 (T a multiple of 16, every sequence T tokens long)
    into a device pool with cf_kv_encode_groups_async, without a host round trip of the values. Group g of
    (sequence s, head h) holds pages 4g..4g+3 of that (s, h). Synchronises once to read the pool end and status."""
    S, H, T, D = keys.shape
    assert values.shape == keys.shape and T % PAGE_TOKENS == 0 and keys.is_contiguous() and values.is_contiguous()
    dev = keys.device
    npg = T // PAGE_TOKENS
    ngr = (npg + GROUP_PAGES - 1) // GROUP_PAGES
    g = torch.arange(S * H * ngr, device=dev, dtype=torch.int64)
    gl = g % ngr
    first = (g // ngr) * npg + gl * GROUP_PAGES
    counts = torch.clamp(npg - gl * GROUP_PAGES, max=GROUP_PAGES).to(torch.int32)
    heads = ((g // ngr) % H).to(torch.int32)
    cont = (gl % 2 == 1).to(torch.uint8)  # groups 2k, 2k + 1 of each (sequence, head) form one chain
    cap = int(A.lib().cf_kv_group_blob_max_bytes(codec, D)) * S * H * ngr
    pool = torch.empty(cap, dtype=torch.uint8, device=dev)
    r = encode_groups_device(codec, keys.view(-1, PAGE_TOKENS, D), values.view(-1, PAGE_TOKENS, D), D, tables, first,
                             counts, pool, 0, heads, None, None, stream, continues=cont)
    st, end = int(r.status.item()), int(r.pool_end.item())
    if st != 0:
        raise A.CfError(st, "cf_kv_encode_groups_async (device status)")
    t_tok = torch.full((S,), T, dtype=torch.int32, device=dev)
    return BatchedKv(codec, S, H, D, ngr, pool[:end], r.offsets.view(S, H, ngr), t_tok, tables)


def build_batched(codec: int, kv_source, seq_count: int, kv_heads: int, seq_tokens: np.ndarray, head_dim: int,
                  tables: np.ndarray | None, device="cuda", keep_host: bool = False,
                  shared: dict | None = None, encoder: str = "host", raw_groups: dict | None = None) -> BatchedKv:
    """Encode and upload page groups. kv_source(s) -> (K, V) fp32 arrays [kv_heads, T_s, D] for sequence s.
    `shared` optionally maps sequence s -> (donor sequence, prefix groups): the first `prefix groups` groups of s are
    the donor's blobs (no copy), modelling refcounted shared-prefix pages. `raw_groups` optionally maps sequence s
    -> n: its first n groups are stored with the INT8 codec (raw symbols, decode-free) inside the pool whatever
    `codec` is; meant for pages many sequences read every step, such as a shared prefix (host encoder only).
    encoder="device" uploads the fp32 pages and seals them with cf_kv_encode_groups_async straight into the device
    pool (same bytes as the host encoder)."""
    seq_tokens = np.asarray(seq_tokens, np.uint32)
    max_groups = int((seq_tokens.max() + GROUP_TOKENS - 1) // GROUP_TOKENS)
    offsets = np.zeros((seq_count, kv_heads, max_groups), np.uint32)
    blobs, at = [], 0
    on_device = encoder == "device"
    if on_device:
        L = A.lib()
        cap = int(L.cf_kv_group_blob_max_bytes(codec, head_dim))
        groups = int(sum(kv_heads * ((int(t) + GROUP_TOKENS - 1) // GROUP_TOKENS) for t in seq_tokens))
        dpool = torch.empty(groups * cap + 16, dtype=torch.uint8, device=device)
        d_tab = None if tables is None else torch.from_numpy(np.ascontiguousarray(tables).ravel()).to(device)
    for s in range(seq_count):
        T = int(seq_tokens[s])
        npg = (T + PAGE_TOKENS - 1) // PAGE_TOKENS
        ngr = (npg + GROUP_PAGES - 1) // GROUP_PAGES
        first = 0
        share = (shared or {}).get(s)
        if share is not None:
            donor, first = share
            offsets[s, :, :first] = offsets[donor, :, :first]
        if first >= ngr:
            continue
        K, V = kv_source(s)
        pad = npg * PAGE_TOKENS - T
        if pad:
            K = np.concatenate([K, np.zeros((kv_heads, pad, head_dim), np.float32)], 1)
            V = np.concatenate([V, np.zeros((kv_heads, pad, head_dim), np.float32)], 1)
        p0 = first * GROUP_PAGES
        Kp = np.ascontiguousarray(K[:, p0 * PAGE_TOKENS:]).reshape(kv_heads * (npg - p0), PAGE_TOKENS, head_dim)
        Vp = np.ascontiguousarray(V[:, p0 * PAGE_TOKENS:]).reshape(kv_heads * (npg - p0), PAGE_TOKENS, head_dim)
        tc = np.full((kv_heads, npg - p0), PAGE_TOKENS, np.uint32)
        if pad:
            tc[:, -1] = PAGE_TOKENS - pad
        gl = np.arange(first, ngr)
        first_page = (np.arange(kv_heads)[:, None] * (npg - p0) + (gl[None, :] - first) * GROUP_PAGES).ravel()
        page_counts = np.broadcast_to(np.minimum(GROUP_PAGES, npg - gl * GROUP_PAGES)[None, :],
                                      (kv_heads, gl.size)).ravel()
        heads = np.repeat(np.arange(kv_heads, dtype=np.uint32), gl.size)
        if on_device:
            if (raw_groups or {}).get(s):
                raise ValueError("raw_groups needs the host encoder")
            cont = np.tile(pair_flags(gl), kv_heads)
            r = encode_groups_device(codec, torch.from_numpy(Kp).to(device), torch.from_numpy(Vp).to(device),
                                     head_dim, d_tab, torch.from_numpy(first_page.astype(np.int64)).to(device),
                                     torch.from_numpy(page_counts.astype(np.int32)).to(device), dpool, at,
                                     torch.from_numpy(heads.view(np.int32)).to(device),
                                     torch.from_numpy(tc.ravel().view(np.int32)).to(device),
                                     continues=torch.from_numpy(cont).to(device))
            if int(r.status.item()) != 0:
                raise A.CfError(int(r.status.item()), "cf_kv_encode_groups_async (device status)")
            offsets[s, :, first:ngr] = r.offsets.cpu().numpy().view(np.uint32).reshape(kv_heads, gl.size)
            at = int(r.pool_end.item())
            continue
        nraw = min(max(int((raw_groups or {}).get(s, 0)) - first, 0), gl.size)
        per_head = [np.arange(h * gl.size, (h + 1) * gl.size) for h in range(kv_heads)]
        for lo, hi, cdc in ((0, nraw, CODEC_INT8), (nraw, gl.size, codec)):
            if hi <= lo:
                continue
            sel = np.concatenate([ph[lo:hi] for ph in per_head])
            cont = np.tile(pair_flags(gl[lo:hi]), kv_heads) if cdc != CODEC_INT8 else None
            blob, offs = encode_groups(cdc, Kp, Vp, head_dim, tables if cdc != CODEC_INT8 else None,
                                       first_page[sel], page_counts[sel], heads[sel], tc.ravel(), continues=cont)
            offsets[s, :, first + lo:first + hi] = (offs + at // 16).reshape(kv_heads, hi - lo)
            blobs.append(blob)
            at += blob.size
    assert at // 16 < 2 ** 32
    if on_device:
        pool = dpool[:max(at, 16)]
        host_pool = pool.cpu().numpy() if keep_host else None
    else:
        host_pool = np.concatenate(blobs) if blobs else np.zeros(16, np.uint8)
        pool = torch.from_numpy(host_pool).to(device)
    t_off = torch.from_numpy(offsets.view(np.int32)).to(device)
    t_tok = torch.from_numpy(seq_tokens.view(np.int32)).to(device)
    t_tab = None if tables is None else torch.from_numpy(np.ascontiguousarray(tables).ravel()).to(device)
    kv = BatchedKv(codec, seq_count, kv_heads, head_dim, max_groups, pool, t_off, t_tok, t_tab)
    if keep_host:
        kv.host_pool, kv.host_offsets, kv.host_tables = host_pool, offsets, tables
    return kv
