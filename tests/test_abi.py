"""The C-ABI library on the CPU (no GPU needed):

  * libchromofold.so exports every function declared in include/chromofold/*.h (C names, plus the reference's C++
    cf_gpu_suffix_array) — and the reference's public/benchmark symbol set;
  * the headers compile as C99 and link (tests/abi/abi_check.c), and every entry point rejects NULL arguments with
    CF_ERR_INVALID_ARGUMENT before touching the device (the reference's NULL-argument contract,
    packaging/conformance.c / chromofold_capability.json "abi_contract");
  * the ctypes mirrors of the ABI structs have the sizes the C compiler gives the header structs.
"""
import ctypes as C
import glob
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "chromofold_amd", "libchromofold.so")
needs_lib = pytest.mark.skipif(not os.path.exists(LIB), reason="libchromofold.so not built")

# the reference's exported surface (include/chromofold/*.h + its benchmark-level extern "C" entry points)
REFERENCE_SYMBOLS = """
cf_access_async cf_rank_async cf_embedding_gather_async cf_kv_attn_fused_async cf_kv_attn_dense_async
cf_rrrw_access_async cf_rrrw_rank_async cf_fm_count_async cf_fm_ranges_async cf_fm_locate_async
cf_kv_validate_paged_attention_desc cf_kv_paged_attention_async cf_kv_validate_page cf_kv_validate_layout
cf_kv_page_resident_bytes cf_kv_cache_memory_stats cf_online_softmax_init cf_online_softmax_accumulate
cf_online_softmax_merge cf_online_softmax_finalize cf_rans_decode_async cf_fused_matmul_async cf_dense_matmul_async
cf_rrr_rank_async cf_rank2_async cf_delta_fetch_async cf_sparse_gather_fused_async cf_sparse_decode_all_async
cf_sparse_gather_async cf_embedding_gather_tpq_async
""".split()


def _declared() -> set[str]:
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "chromofold", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w ]*?[\s\*]+(cf_\w+)\s*\(", src, flags=re.M):
            names.add(m.group(1))
    return names


def _exported() -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


@needs_lib
def test_every_declared_symbol_is_exported():
    declared, exported = _declared(), _exported()
    assert len(declared) >= 40
    c_names = {n for n in declared if n != "cf_gpu_suffix_array"}
    assert not (c_names - exported), sorted(c_names - exported)
    assert any(n.startswith("_Z") and "cf_gpu_suffix_array" in n for n in exported)
    assert not (set(REFERENCE_SYMBOLS) - exported), sorted(set(REFERENCE_SYMBOLS) - exported)


@needs_lib
@pytest.mark.skipif(shutil.which("gcc") is None, reason="no C compiler")
def test_c_headers_link_and_null_contract(tmp_path):
    exe = str(tmp_path / "abi_check")
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "abi", "abi_check.c"), "-L", os.path.dirname(LIB), "-lchromofold",
                    "-Wl,-rpath," + os.path.dirname(LIB), "-o", exe], check=True, capture_output=True, timeout=120)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASS" in r.stdout
    from chromofold_amd import _abi as A
    from chromofold_amd import kv, qw, search, sealkv
    mirrors = {"cf_wavelet_view": A.cf_wavelet_view, "cf_rrrw_view": A.cf_rrrw_view, "cf_fm_view": A.cf_fm_view,
               "cf_kv_device_page": A.cf_kv_device_page, "cf_kv_paged_attention_desc": A.cf_kv_paged_attention_desc,
               "cf_kv_batched_desc": kv.cf_kv_batched_desc, "cf_qw_matrix": qw.cf_qw_matrix,
               "cf_rrrw_file_header": search.cf_rrrw_file_header, "cf_fm_file_header": search.cf_fm_file_header,
               "cf_fm_file_arrays": search.cf_fm_file_arrays,
               "cf_device_tensor_view": sealkv.cf_device_tensor_view,
               "cf_device_page_descriptor": sealkv.cf_device_page_descriptor,
               "cf_device_seal_counters": sealkv.cf_device_seal_counters,
               "cf_device_kv_counters": sealkv.cf_device_kv_counters,
               "cf_ms_page_publication": sealkv.cf_ms_page_publication,
               "cf_ms_batch_item": sealkv.cf_ms_batch_item, "cf_ms_cuda_counters": sealkv.cf_ms_cuda_counters,
               "cf_attention_runtime_config": sealkv.cf_attention_runtime_config,
               "cf_attention_batch_item": sealkv.cf_attention_batch_item,
               "cf_attention_counters": sealkv.cf_attention_counters}
    sizes = dict(re.findall(r"^sizeof (\w+) (\d+)$", r.stdout, flags=re.M))
    assert set(sizes) == set(mirrors)
    for name, cls in mirrors.items():
        assert C.sizeof(cls) == int(sizes[name]), name


@needs_lib
def test_hip_imports_resolve_in_torchs_runtime():
    """The library is loaded after torch, into torch's own libamdhip64 (ROCm 7.0 in this image, older than the
    hipcc that builds the library): every versioned HIP symbol the library imports must be exported by that
    runtime at that version, or the library fails to load on the GPU box."""
    import torch
    rt = glob.glob(os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so*"))
    if not rt:
        pytest.skip("torch ships no libamdhip64 here")
    need = subprocess.run(["nm", "-D", "--undefined-only", LIB], capture_output=True, text=True, check=True).stdout
    have = subprocess.run(["nm", "-D", "--defined-only", rt[0]], capture_output=True, text=True, check=True).stdout
    have_set = {line.split()[-1].replace("@@", "@") for line in have.splitlines() if line.strip()}
    missing = [s for s in (line.split()[-1] for line in need.splitlines() if "@hip_" in line) if s not in have_set]
    assert not missing, missing
