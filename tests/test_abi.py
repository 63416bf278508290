"""CPU checks of the C-ABI library: it loads, exports every function that
include/minirun_hip.h declares, and rejects bad arguments with named errors
without touching a GPU (argument checks run before any HIP call)."""
import ctypes as C
import os
import re

import pytest

import minirun_hip as M

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names += re.findall(r"\b(mr_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = M.load()
    names = declared_functions()
    assert "mr_mla_decode" in names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert set(names) <= set(M.SIGNATURES), "binding lacks a signature for a declared function"


def test_version_and_error_string():
    assert M.version().startswith("minirun-hip")
    assert isinstance(M.last_error(), str)


def test_decode_rejects_bad_arguments_before_any_gpu_call():
    lib = M.load()
    a = M.DecodeArgs()
    a.batch, a.heads, a.n_ctx, a.kv_rank, a.rope_dim, a.scale = 1, 16, 512, 4096, 64, 0.07
    assert lib.mr_mla_decode(C.byref(a), None) == M.INVALID_SHAPE  # widths beyond the any-width kernel
    assert "kv_rank" in M.last_error()
    a.kv_rank, a.rope_dim = 256, 600
    assert lib.mr_mla_decode(C.byref(a), None) == M.INVALID_SHAPE and "rope_dim" in M.last_error()
    a.rope_dim = 64
    assert lib.mr_mla_decode(C.byref(a), None) == M.INVALID_ARGUMENT  # other widths: on to the pointer checks
    a.kv_rank = 512
    a.scale = -1.0
    assert lib.mr_mla_decode(C.byref(a), None) == M.INVALID_SHAPE
    a.scale = 0.07
    assert lib.mr_mla_decode(C.byref(a), None) == M.INVALID_ARGUMENT  # NULL pointers
    assert lib.mr_mla_decode(None, None) == M.INVALID_ARGUMENT


def test_workspace_size_is_deterministic_and_covers_partials():
    lib = M.load()
    a = M.DecodeArgs()
    a.batch, a.heads, a.n_ctx, a.kv_rank, a.rope_dim, a.scale = 1, 128, 32768, 512, 64, 0.07
    a.num_splits = 64
    n = lib.mr_mla_decode_workspace_size(C.byref(a))
    # per (split, head): O / l as 512 bf16 plus (m, l) as two fp32
    assert n >= 64 * 128 * (512 * 2 + 2 * 4)
    assert n == lib.mr_mla_decode_workspace_size(C.byref(a))


def test_any_width_workspace_sizes():
    # widths the split kernel does not take have no split partials: the
    # workspace holds only the index checks' words (and long lists' tables)
    lib = M.load()
    a = M.DecodeArgs()
    a.batch, a.heads, a.n_ctx, a.kv_rank, a.rope_dim, a.scale = 2, 4, 37, 16, 4, 12 ** -0.5
    assert lib.mr_mla_decode_workspace_size(C.byref(a)) == 0
    a.indices, a.n_idx = 1, 12  # any non-NULL pointer: sizing reads no memory
    assert lib.mr_mla_decode_workspace_size(C.byref(a)) == lib.mr_validate_indices_workspace_size(2, 12)
    a.flags = M.DECODE_UNCHECKED
    assert lib.mr_mla_decode_workspace_size(C.byref(a)) == 0
    p = M.PrefillArgs()
    p.tokens, p.n_ctx, p.heads = 5, 9, 4
    p.qk_nope_dim, p.qk_rope_dim, p.v_head_dim, p.kv_rank = 8, 4, 8, 16
    assert lib.mr_mla_prefill_workspace_size(C.byref(p)) == -(-(9 * 4 * (8 + 8) * 4) // 256) * 256
    p.qk_nope_dim, p.qk_rope_dim, p.v_head_dim, p.kv_rank = 128, 64, 128, 512
    assert lib.mr_mla_prefill_workspace_size(C.byref(p)) == 9 * 4 * 256 * 2 // 256 * 256 + (256 if 9 * 4 * 512 % 256 else 0)


def test_prefill_width_limits():
    lib = M.load()
    p = M.PrefillArgs()
    p.tokens, p.n_ctx, p.heads, p.scale = 5, 9, 4, 0.2
    p.qk_nope_dim, p.qk_rope_dim, p.v_head_dim, p.kv_rank = 8, 4, 8, 4096
    assert lib.mr_mla_prefill(C.byref(p), None) == M.INVALID_SHAPE and "kv_rank" in M.last_error()
    p.kv_rank, p.v_head_dim = 16, 0
    assert lib.mr_mla_prefill(C.byref(p), None) == M.INVALID_SHAPE
    p.v_head_dim = 8
    assert lib.mr_mla_prefill(C.byref(p), None) == M.INVALID_ARGUMENT  # NULL pointers


def test_validate_indices_rejects_oversize_without_gpu():
    lib = M.load()
    st = lib.mr_validate_indices(None, 1, (1 << 22) + 1, 10, None, 0, None, None, None)
    assert st == M.INVALID_SHAPE
    assert lib.mr_validate_indices(None, 1, 1 << 22, 10, None, 0, None, None, None) == M.INVALID_ARGUMENT


def test_validate_workspace_holds_long_list_tables():
    # lists of up to 10176 entries are checked in LDS (the workspace holds
    # the results only); longer ones keep one hash table per token there,
    # at least 1.6 slots of 8 bytes per entry
    lib = M.load()
    small = lib.mr_validate_indices_workspace_size(4, 10176)
    assert small == 256
    big = lib.mr_validate_indices_workspace_size(4, 10177)
    assert big >= 256 + 4 * 8 * int(1.6 * 10177)
    assert lib.mr_validate_indices_workspace_size(2, 300000) >= 2 * 8 * int(1.6 * 300000)


def test_sparse_decode_bounds_the_index_count_without_gpu():
    # a gathered split stages at most 512 indices and the combine merges at
    # most 1024 splits: longer lists are refused before any launch
    lib = M.load()
    a = M.DecodeArgs()
    a.batch, a.heads, a.n_ctx, a.kv_rank, a.rope_dim, a.scale = 1, 128, 1 << 20, 512, 64, 0.07
    a.indices = 256  # never dereferenced: the shape checks come first
    a.n_idx = 512 * 1024 + 1
    assert lib.mr_mla_decode(C.byref(a), None) == M.INVALID_SHAPE and "exceeds 524288" in M.last_error()
    a.flags = M.DECODE_UNCHECKED
    assert lib.mr_mla_decode(C.byref(a), None) == M.INVALID_SHAPE
    a.n_idx = 9000
    assert lib.mr_mla_decode(C.byref(a), None) == M.INVALID_ARGUMENT  # past the shape checks: NULL q
    # checked lists of any length the call takes: the checks add their
    # tables to the workspace once a list is too long for LDS
    a.flags = 0
    assert lib.mr_mla_decode(C.byref(a), None) == M.INVALID_ARGUMENT
    a.n_idx = 512 * 1024
    assert lib.mr_mla_decode(C.byref(a), None) == M.INVALID_ARGUMENT
    a.index_status = 4096  # never dereferenced: the workspace size only
    a.n_idx = 8320
    w_lds = lib.mr_mla_decode_workspace_size(C.byref(a))
    a.n_idx = 20000
    w_tab = lib.mr_mla_decode_workspace_size(C.byref(a))
    assert w_tab - w_lds >= 8 * int(1.6 * 20000)


def test_prefill_rejects_bad_arguments_before_any_gpu_call():
    lib = M.load()
    a = M.PrefillArgs()
    a.tokens, a.n_ctx, a.heads = 4096, 4096, 128
    a.qk_nope_dim, a.qk_rope_dim, a.v_head_dim, a.kv_rank = 128, 64, 128, 4096
    a.scale = 192 ** -0.5
    assert lib.mr_mla_prefill(C.byref(a), None) == M.INVALID_SHAPE  # beyond the any-width kernels
    assert "kv_rank" in M.last_error()
    a.kv_rank = 512
    a.n_ctx = 100
    assert lib.mr_mla_prefill(C.byref(a), None) == M.INVALID_SHAPE
    assert "cover" in M.last_error()
    a.n_ctx = 4096
    assert lib.mr_mla_prefill(C.byref(a), None) == M.INVALID_ARGUMENT  # NULL pointers
    assert lib.mr_mla_prefill(None, None) == M.INVALID_ARGUMENT
    assert lib.mr_mla_prefill_workspace_size(C.byref(a)) == 4096 * 128 * 512


def _dense_desc(addr, out_f, in_f, dtype=M.BF16):
    p = M.ProjectionDesc()
    p.kind = M.PROJ_DENSE
    p.dense.weight, p.dense.dtype, p.dense.out_features, p.dense.in_features, p.dense.row_stride = \
        addr, dtype, out_f, in_f, in_f
    return p


def _k3_prefill_block_args(T=64, position=0):
    """K3 widths with placeholder device addresses: the checks read no memory."""
    a = M.PrefillBlockArgs()
    a.tokens, a.hidden, a.q_lora_rank, a.heads = T, 7168, 1536, 96
    a.qk_nope_dim, a.qk_rope_dim, a.v_head_dim, a.kv_rank = 128, 64, 128, 512
    a.eps, a.scale = 1e-6, 192 ** -0.5
    base = 1 << 32
    a.x, a.x_token_stride = base, 7168
    a.q_a_norm_w, a.kv_a_norm_w, a.norm_w_dtype = base + 0x100000, base + 0x200000, M.BF16
    a.q_a = _dense_desc(base + 0x1000000, 1536, 7168)
    a.q_b = _dense_desc(base + 0x2000000, 96 * 192, 1536)
    a.kv_a = _dense_desc(base + 0x3000000, 576, 7168)
    a.kv_b = _dense_desc(base + 0x4000000, 96 * 256, 512)
    a.o_proj = _dense_desc(base + 0x5000000, 7168, 96 * 128)
    a.g_proj = _dense_desc(base + 0x6000000, 96 * 128, 7168)
    a.cache_latent, a.latent_row_stride = base + 0x10000000, 576
    a.cache_rope, a.rope_row_stride = base + 0x10000000 + 1024, 576
    a.position, a.capacity = position, position + T
    a.out, a.out_token_stride = base + 0x20000000, 7168
    a.workspace = base + 0x40000000
    a.workspace_bytes = M.load().mr_mla_prefill_block_workspace_size(C.byref(a))
    return a


def test_prefill_block_workspace_layout():
    lib = M.load()
    a = _k3_prefill_block_args(T=64, position=30)
    al = lambda n: -(-n // 256) * 256
    T, P = 64, 94
    want = (al(T * 1536 * 2) * 2 + al(T * 96 * 192 * 2) + al(T * 576 * 2) + al(T * 96 * 128 * 2) * 2
            + al(P * 96 * 256 * 2))
    assert a.workspace_bytes == want
    a.input_norm_w = 1 << 40  # an input norm stages the normed rows
    assert lib.mr_mla_prefill_block_workspace_size(C.byref(a)) == want + al(T * 7168 * 2)
    assert lib.mr_mla_prefill_block_workspace_size(None) == 0


def test_prefill_block_rejects_bad_arguments_before_any_gpu_call():
    lib = M.load()
    call = lambda a: lib.mr_mla_prefill_block(C.byref(a), None)
    assert lib.mr_mla_prefill_block(None, None) == M.INVALID_ARGUMENT
    a = _k3_prefill_block_args()
    a.capacity = 63
    assert call(a) == M.INVALID_SHAPE and "capacity" in M.last_error()
    a = _k3_prefill_block_args()
    a.qk_rope_dim = 63
    assert call(a) == M.INVALID_SHAPE and "even" in M.last_error()
    a = _k3_prefill_block_args()
    a.q_b = _dense_desc(1 << 33, 96 * 192 + 8, 1536)
    assert call(a) == M.INVALID_SHAPE and "q_b_proj" in M.last_error()
    a = _k3_prefill_block_args()
    a.kv_b = _dense_desc(1 << 33, 96 * 256, 512, M.F32)
    assert call(a) == M.INVALID_DTYPE and "kv_b_proj" in M.last_error()
    a = _k3_prefill_block_args()
    a.workspace_bytes -= 256
    assert call(a) == M.WORKSPACE_TOO_SMALL
    a = _k3_prefill_block_args()
    a.rope_cos = 1 << 34  # one rotary table without the other
    assert call(a) == M.INVALID_ARGUMENT
    a = _k3_prefill_block_args()
    a.latent_row_stride = 580  # the attention's fixed-width kernels step 16-byte rows
    assert call(a) == M.INVALID_ARGUMENT and "multiples of 8" in M.last_error()
    a = _k3_prefill_block_args()
    a.kv_rank, a.kv_a, a.kv_b = 4096, _dense_desc(1 << 33, 4160, 7168), _dense_desc(1 << 34, 96 * 256, 4096)
    a.latent_row_stride = a.rope_row_stride = 4160
    assert call(a) == M.INVALID_SHAPE and "kv_rank" in M.last_error()


def test_header_compiles_as_c_and_host_entry_points_work_from_c(tmp_path):
    """include/minirun_hip.h as a C11 translation unit (what a Swift module
    map imports): a C program links the library and checks the host-side
    entry points.  Built in a temporary directory; no GPU call."""
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    lib_dir = os.path.dirname(M.LIB_PATH)
    exe = str(tmp_path / "abi_from_c")
    src = os.path.join(ROOT, "tests", "c_abi", "abi_from_c.c")
    r = subprocess.run([cc, "-std=c11", "-Wall", "-Wextra", "-Werror", "-pedantic", "-I", os.path.join(ROOT, "include"),
                        src, "-o", exe, "-L", lib_dir, "-lminirun_hip", f"-Wl,-rpath,{lib_dir}"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "abi_from_c: ok" in r.stdout
