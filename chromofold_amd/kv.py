"""Host-side mirror of the compressed paged-KV interface.

Two entry points are mirrored:
  * the batched multi-sequence decode of include/chromofold/kv_codec_ext.h (INT8 / RANS_HYBRID page blobs in one
    device pool, per-(sequence, head) page tables, split-context workspace) — the benchmark path;
  * the legacy single-sequence seam cf_kv_paged_attention_async of include/chromofold/kv_cuda.h (see legacy.py).

Encoding happens on the host through the library's C encoder (cf_kv_encode_groups); pools, page tables, queries
and outputs live in HBM as torch tensors. Every launch goes through libchromofold.so.
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
EXT_ABI_VERSION = 2
GROUP_PAGES = 4
GROUP_TOKENS = PAGE_TOKENS * GROUP_PAGES


class cf_kv_batched_desc(C.Structure):
    _fields_ = [("struct_size", A.U32), ("abi_version", A.U32), ("codec", A.U32), ("seq_count", A.U32),
                ("kv_head_count", A.U32), ("query_head_count", A.U32), ("head_dim", A.U32), ("max_groups", A.U32),
                ("pool", A.P), ("group_offsets", A.P), ("seq_tokens", A.P), ("query_pos", A.P), ("tables", A.P),
                ("queries", A.P), ("output", A.P), ("softmax_scale", A.F32), ("splits", A.U32),
                ("workspace", A.P), ("workspace_bytes", A.U64)]


A.declare("cf_kv_encode_groups", A.I32, [A.U32, A.P, A.P, A.U64, A.P, A.P, A.P, A.U32, A.P, A.P, A.P, A.U64, A.U64,
                                         A.P, A.P, A.U32])
A.declare("cf_kv_encode_group", A.I32, [A.U32, A.P, A.P, A.U32, A.P, A.U32, A.P, A.P, A.U32, A.U32, A.P, A.U64, A.P])
A.declare("cf_kv_rans_build_table", A.I32, [A.P, A.P])
A.declare("cf_kv_rans_page_histogram", A.I32, [A.P, A.U32, A.U32, A.P])
A.declare("cf_kv_group_blob_max_bytes", A.U64, [A.U32, A.U32])
A.declare("cf_kv_batched_workspace_bytes", A.U64, [A.P])
A.declare("cf_kv_validate_batched_desc", A.I32, [A.P])
A.declare("cf_kv_paged_attention_batched_async", A.I32, [A.P, A.P])


def _np_ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def build_table(pages: np.ndarray) -> np.ndarray:
    """Table blob from the joint high-part histogram of sample pages [n, tokens<=16, D] (fp32)."""
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
                  token_counts: np.ndarray | None = None, threads: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """Encode page groups of page-major pages keys/values [n_pages, 16, D] -> (blob bytes, offsets/16)."""
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
    st = L.cf_kv_encode_groups(codec, _np_ptr(keys), _np_ptr(values), n, _np_ptr(first_page), _np_ptr(page_counts),
                               _np_ptr(tc), head_dim, _np_ptr(tables), _np_ptr(hd), _np_ptr(pool), cap, 0,
                               _np_ptr(offs), C.byref(end), threads)
    A.check(st, "cf_kv_encode_groups")
    return pool[:end.value], offs


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
             splits: int = 0) -> cf_kv_batched_desc:
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
        need = int(A.lib().cf_kv_batched_workspace_bytes(C.byref(d)))
        if need:
            if self.workspace is None or self.workspace.numel() < need:
                self.workspace = torch.empty(need, dtype=torch.uint8, device=self.pool.device)
            d.workspace = self.workspace.data_ptr()
            d.workspace_bytes = self.workspace.numel()
        return d

    def attention(self, queries: torch.Tensor, output: torch.Tensor, query_pos: torch.Tensor,
                  softmax_scale: float, splits: int = 0, stream=None, desc: cf_kv_batched_desc | None = None):
        d = desc if desc is not None else self.desc(queries, output, query_pos, softmax_scale, splits)
        s = (stream if stream is not None else torch.cuda.current_stream()).cuda_stream
        A.check(A.lib().cf_kv_paged_attention_batched_async(C.byref(d), s), "cf_kv_paged_attention_batched_async")


def build_batched(codec: int, kv_source, seq_count: int, kv_heads: int, seq_tokens: np.ndarray, head_dim: int,
                  tables: np.ndarray | None, device="cuda", keep_host: bool = False,
                  shared: dict | None = None) -> BatchedKv:
    """Encode and upload page groups. kv_source(s) -> (K, V) fp32 arrays [kv_heads, T_s, D] for sequence s.
    `shared` optionally maps sequence s -> (donor sequence, prefix groups): the first `prefix groups` groups of s are
    the donor's blobs (no copy), modelling refcounted shared-prefix pages."""
    seq_tokens = np.asarray(seq_tokens, np.uint32)
    max_groups = int((seq_tokens.max() + GROUP_TOKENS - 1) // GROUP_TOKENS)
    offsets = np.zeros((seq_count, kv_heads, max_groups), np.uint32)
    blobs, at = [], 0
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
        blob, offs = encode_groups(codec, Kp, Vp, head_dim, tables, first_page, page_counts, heads, tc.ravel())
        offsets[s, :, first:ngr] = (offs + at // 16).reshape(kv_heads, gl.size)
        blobs.append(blob)
        at += blob.size
    host_pool = np.concatenate(blobs) if blobs else np.zeros(16, np.uint8)
    assert at // 16 < 2 ** 32
    pool = torch.from_numpy(host_pool).to(device)
    t_off = torch.from_numpy(offsets.view(np.int32)).to(device)
    t_tok = torch.from_numpy(seq_tokens.view(np.int32)).to(device)
    t_tab = None if tables is None else torch.from_numpy(np.ascontiguousarray(tables).ravel()).to(device)
    kv = BatchedKv(codec, seq_count, kv_heads, head_dim, max_groups, pool, t_off, t_tok, t_tab)
    if keep_host:
        kv.host_pool, kv.host_offsets, kv.host_tables = host_pool, offsets, tables
    return kv
