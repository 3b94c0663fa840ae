"""ctypes binding of librlt_mi355x.so (the C ABI declared in include/rlt_mi355x.h),
and the loader of the C++ torch operators over it (``_C.so``, ``ops()``).

There is no fallback: if a library is missing or the device is not a ROCm
GPU, every op raises.  Build it with ``python vllm-rlt_amd/build.py`` (or
``__graft_entry__.build()``).
"""

import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librlt_mi355x.so")
OPS_PATH = os.path.join(HERE, "_C.so")

RLT_F32, RLT_F16, RLT_BF16, RLT_FP8_E4M3 = 0, 1, 2, 3
_DTYPE_CODE = {
    torch.float32: RLT_F32,
    torch.float16: RLT_F16,
    torch.bfloat16: RLT_BF16,
    torch.float8_e4m3fn: RLT_FP8_E4M3,
}
_STATUS = {
    1: "invalid argument",
    2: "unsupported configuration",
    3: "workspace too small",
    4: "kernel launch failed",
}

_i32, _i64, _sz, _p = ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p

# the interface version of include/rlt_mi355x.h these signatures were written for
RLT_ATTN_COMPENSATE = 1
ABI_VERSION = 4

_SIGNATURES = {
    "rlt_abi_version": (ctypes.c_int, []),
    "rlt_paged_attention_workspace_size": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "rlt_paged_attention_uses_mfma": (ctypes.c_int, [_i32, _i32, _i32]),
    "rlt_paged_attention_uses_prefill": (ctypes.c_int, [_i32, _i32, _i32, _i32]),
    "rlt_paged_attention": (ctypes.c_int, [
        _p, _i64, _i64,                 # q
        _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,  # k, v, strides
        _i32,                           # num_blocks
        _p, _i64, _i32,                 # tables
        _p, _p, _i32, _i32, _i32,       # lengths, cu, num_seqs, max_q_len, num_q_rows
        _p, _p, _i32, _i64, _i64, _i64,  # scales
        _i32, _i32, _i32, _i32,         # hq, hkv, head_dim, block_size
        _i32, _i32, _i32,               # q dtype, kv dtype, window
        _p, _i64, _i64,                 # out
        _p, _sz, _p,                    # workspace, bytes, stream
    ]),
    "rlt_paged_attention_rows": (ctypes.c_int, [
        _p, _i64, _i64,                 # q
        _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,  # k, v, strides
        _i32,                           # num_blocks
        _p, _i64, _i32,                 # tables
        _p, _p,                         # lengths, row lengths
        _p, _i32, _i32, _i32,           # cu, num_seqs, max_q_len, num_q_rows
        _p, _p, _i32, _i64, _i64, _i64,  # scales
        _i32, _i32, _i32, _i32,         # hq, hkv, head_dim, block_size
        _i32, _i32, _i32, _i32,         # q dtype, kv dtype, window, flags
        _p, _i64, _i64,                 # out
        _p, _sz, _p,                    # workspace, bytes, stream
    ]),
    "rlt_paged_attention_store_scaled": (ctypes.c_int, [
        _p, _i64, _i64,                 # q
        _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i32,  # pools, strides, blocks
        _p, _i64, _i32,                 # tables, stride, width
        _p, _p, _p,                     # lengths, row lengths, cu
        _i32, _i32, _i32,               # num_seqs, max_q_len, num_q_rows
        _p, _p, _i32, _i64, _i64, _i64,  # scales
        _i32, _i32, _i32, _i32,         # hq, hkv, head_dim, block_size
        _i32, _i32, _i32,               # q dtype, kv dtype, flags
        _p, _p, _i64, _i64,             # new k, v, row / head strides
        _p, _i64, _i64,                 # out
        _p, _sz, _p,                    # workspace, bytes, stream
    ]),
    "rlt_paged_attention_store": (ctypes.c_int, [
        _p, _i64, _i64,                 # q
        _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i32,  # pools, strides, blocks
        _p, _i64, _i32, _p,             # tables, stride, width, lengths
        _p, _i32, _i32, _i32,           # cu, num_seqs, max_q_len, num_q_rows
        _i32, _i32, _i32, _i32, _i32,   # hq, hkv, head_dim, block_size, dtype
        _p, _p, _i64, _i64,             # new k, v, row / head strides
        _p, _i64, _i64,                 # out
        _p, _sz, _p,                    # workspace, bytes, stream
    ]),
    "rlt_merge_random_round": (ctypes.c_int, [
        _p, _i64, _p, _p, _p, _p, _i64,  # target, rows, accepted, next, starts, inputs, n
        _p, _i32, _p, _p, _p, _p, _i64,  # tokens, width, accepted, final, error, requests, r
        _p, _p, _p, _i64,                # verify rows, ranks, offsets, count
        _p, _p, _p, _p, _p, _p, _p,      # outputs, stream
    ]),
    "rlt_speculative_accept_workspace_size": (_sz, [_i64, _i32, _i64]),
    "rlt_speculative_accept": (ctypes.c_int, [
        _p, _p, _p, _p, _p, _p, _i64, _i32, _i64, _p, _p, _p, _p, _p, _sz, _p]),
    "rlt_speculative_accept_noalloc_max_bytes": (_sz, []),
    "rlt_speculative_accept_noalloc": (ctypes.c_int, [
        _p, _p, _p, _p, _p, _p, _i64, _i32, _i64, _p, _p, _p, _p, _p]),
    "rlt_rejection_sample_workspace_size": (_sz, [_i64, _i64, _i32]),
    "rlt_rejection_sample": (ctypes.c_int, [
        _p, _p, _p, _p, _p, _i64, _i32, _i64, _i32, _p, _p, _p, _p, _sz, _p]),
    "rlt_categorical_workspace_size": (_sz, [_i64, _i64]),
    "rlt_categorical": (ctypes.c_int, [_p, _p, _i64, _i64, _p, _p, _p, _sz, _p]),
    "rlt_row_mass_workspace_size": (_sz, [_i64, _i64]),
    "rlt_row_mass_f32": (ctypes.c_int, [_p, _i64, _i64, _p, _p, _sz, _p]),
    "rlt_probabilities_workspace_size": (_sz, [_i64, _i64, _i64]),
    "rlt_batched_probabilities": (ctypes.c_int, [
        _p, _i32, _i64, _i64, _i64, _p, _p, _p, _i64, _i32, _p, _i64, _p, _sz, _p]),
    "rlt_propose_drafts_workspace_size": (_sz, [_i64, _i64, _i64]),
    "rlt_propose_drafts": (ctypes.c_int, [
        _p, _i32, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _i64, _i32, _p, _p, _i64, _p, _p, _sz,
        _p]),
    "rlt_verify_distributions": (ctypes.c_int, [
        _p, _i32, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _i64, _i32, _p, _i64, _p, _p, _sz,
        _p]),
    "rlt_verify_accept_workspace_size": (_sz, [_i64, _i32, _i64]),
    "rlt_verify_accept": (ctypes.c_int, [
        _p, _i32, _i64, _p, _p, _p, _i64, _i32, _p, _p, _p, _p, _p, _i64, _i32, _i64, _p, _p, _p,
        _p, _p, _p, _p, _sz, _p]),
    "rlt_greedy_accept": (ctypes.c_int, [
        _p, _p, _p, _i32, _i64, _i64, _i32, _i64, _p, _p, _p, _p]),
    "rlt_kv_store": (ctypes.c_int, [
        _p, _p, _i64, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _i64, _i32,
        _p, _p, _p, _p, _i64, _i32, _i32, _i32, _p]),
    "rlt_kv_store_fp8": (ctypes.c_int, [
        _p, _p, _i32, _i64, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _p,
        _i64, _i64, _i64, _i64, _i32, _p, _p, _p, _p, _i64, _i32, _i32, _i32,
        ctypes.c_float, _p]),
    "rlt_kv_finalize": (ctypes.c_int, [
        _p, _i64, _p, _i64, _i32, _i32, _i32, _i32, _i64, _p, _p, _i64, _i64, _i64,
        _i64, _i32, _p]),
    "rlt_route_slots": (ctypes.c_int, [_p, _p, _i64, _i64, _p]),
    "rlt_route_metadata": (ctypes.c_int, [
        _p, _p, _i64, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p, _i64, _i32, _i64, _i64, _p]),
    "rlt_route_gather": (ctypes.c_int, [
        _p, _i64, _i64, _p, _p, _i64, _i64, _i64, _i64, _i32, _p]),
    "rlt_route_scatter": (ctypes.c_int, [
        _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _i32, _p]),
    "rlt_route_gather_segments": (ctypes.c_int, [
        _p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _i64, _i32, _p]),
    "rlt_route_scatter_segments": (ctypes.c_int, [
        _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i32, _p]),
    "rlt_expand_kv_addresses": (ctypes.c_int, [
        _p, _p, _p, _i64, _i32, _i32, _p, _p, _i64, _p]),
    "rlt_depth_tables": (ctypes.c_int, [
        _p, _i64, _i64, _i32, _i32, _p, _p, _p, _i32, _p, _i64, _p, _p, _p, _i64, _p]),
}

EXPORTED = tuple(_SIGNATURES)

_lib = None


def library():
    """Load the shared library once; raise if it is absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python vllm-rlt_amd/build.py`; "
                "there is no fallback implementation")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        found = lib.rlt_abi_version()
        if found != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} implements C ABI version {found}, these bindings "
                               f"version {ABI_VERSION}: rebuild the library")
        _lib = lib
    return _lib


_ops_loaded = False


def ops():
    """``torch.ops.rlt_mi355x`` with the C++ operators of ``_C.so`` (csrc/torch_bindings.cpp)
    registered; raise if the extension is absent."""
    global _ops_loaded
    if not _ops_loaded:
        if not os.path.exists(OPS_PATH):
            raise RuntimeError(
                f"{OPS_PATH} is missing: build it with `python vllm-rlt_amd/build.py`; "
                "there is no fallback implementation")
        library()  # the C ABI it links against, from this directory
        torch.ops.load_library(OPS_PATH)
        _ops_loaded = True
    return torch.ops.rlt_mi355x


def dtype_code(dtype):
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None


def check(status, what):
    if status != 0:
        raise RuntimeError(f"{what}: {_STATUS.get(status, f'status {status}')}")


def require_gpu(*tensors):
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError("the MI355X kernels require ROCm device tensors")


def stream_of(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def workspace(nbytes, device):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
