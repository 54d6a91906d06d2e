"""ctypes declarations for include/loom_infer_hip.h (libloom_infer_hip.so)."""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# LOOM_INFER_HIP_LIB selects another build of the same library (for example an
# instrumented or tuning build); the default is the in-tree build.
LIB_PATH = os.environ.get("LOOM_INFER_HIP_LIB") or os.path.join(
    os.path.dirname(_HERE), "lib", "libloom_infer_hip.so")

u64, i32, u32, f32, vp = C.c_uint64, C.c_int32, C.c_uint32, C.c_float, C.c_void_p


class Error(C.Structure):
    _fields_ = [("code", i32), ("hip_status", i32), ("operand", C.c_char_p),
                ("fields", C.c_int64 * 4), ("value", C.c_double), ("message", C.c_char * 256)]


class PagedDecodeSpec(C.Structure):
    _fields_ = [("batch_size", u64), ("max_num_pages", u64), ("num_query_heads", u64),
                ("num_kv_heads", u64), ("softmax_scale", f32), ("kv_layout", u32),
                ("kv_dtype", u32), ("page_size", u32)]


class RopeAppendSpec(C.Structure):
    _fields_ = [("paged", PagedDecodeSpec)]


class RopeAppendTokensSpec(C.Structure):
    _fields_ = [("paged", PagedDecodeSpec), ("tokens", u64), ("max_tokens", u64)]


class Handle(C.Structure):
    _fields_ = [("set_id", u64), ("slot", u64)]


class PagedDecodePlanOptions(C.Structure):
    _fields_ = [("max_total_pages", u64), ("teams", u32), ("flags", u32)]


class PagedDecodePlanInfo(C.Structure):
    _fields_ = [("spec", PagedDecodeSpec), ("algorithm", i32), ("teams", u32),
                ("group_tile", u32), ("group_tiles", u32), ("max_total_pages", u64),
                ("state_slots", u64), ("workspace_bytes", u64), ("header_bytes", u64),
                ("block_threads", u32), ("grid_blocks", u32), ("device_cus", u32),
                ("flags", u32)]


class PagedDecodeArgs(C.Structure):
    _fields_ = [(n, Handle) for n in ("query", "key_pages", "value_pages", "page_indptr",
                                      "page_indices", "last_page_len", "output", "lse",
                                      "workspace", "kv_scales")]


class Bf16PagedBatchDecodeArgs(C.Structure):
    _fields_ = [(n, Handle) for n in ("query", "key_pages", "value_pages", "page_indptr",
                                      "page_indices", "last_page_len", "output", "lse")]


class SingleDecodeSpec(C.Structure):
    _fields_ = [("kv_len", u64), ("num_query_heads", u64), ("num_kv_heads", u64),
                ("softmax_scale", f32)]


class SingleDecodeSplitKSpec(C.Structure):
    _fields_ = [("decode", SingleDecodeSpec), ("partitions", u64)]


class SingleDecodeArgs(C.Structure):
    _fields_ = [(n, Handle) for n in ("query", "key", "value", "output", "lse")]


class SingleDecodeSplitKArgs(C.Structure):
    _fields_ = [(n, Handle) for n in ("query", "key", "value", "workspace", "output", "lse")]


class PagedPrefillSpec(C.Structure):
    _fields_ = [("batch_size", u64), ("nnz_qo", u64), ("max_num_pages", u64),
                ("num_query_heads", u64), ("num_kv_heads", u64), ("softmax_scale", f32),
                ("kv_layout", u32), ("page_size", u32), ("kv_dtype", u32)]


class PagedPrefillPlanOptions(C.Structure):
    _fields_ = [("waves", u32), ("flags", u32)]


class PagedPrefillPlanInfo(C.Structure):
    _fields_ = [("spec", PagedPrefillSpec), ("algorithm", i32), ("waves", u32),
                ("row_tiles", u64), ("block_threads", u32), ("grid_blocks", u64),
                ("flags", u32)]


class PagedPrefillArgs(C.Structure):
    _fields_ = [(n, Handle) for n in ("query", "key_pages", "value_pages", "qo_indptr",
                                      "page_indptr", "page_indices", "last_page_len",
                                      "output", "lse", "kv_scales")]


class RaggedPrefillSpec(C.Structure):
    _fields_ = [("batch_size", u64), ("nnz_qo", u64), ("nnz_kv", u64), ("num_query_heads", u64),
                ("num_kv_heads", u64), ("softmax_scale", f32)]


class RaggedPrefillPlanInfo(C.Structure):
    _fields_ = [("spec", RaggedPrefillSpec), ("algorithm", i32), ("waves", u32),
                ("row_tiles", u64), ("block_threads", u32), ("grid_blocks", u64),
                ("workspace_numel", u64)]


class RaggedPrefillArgs(C.Structure):
    _fields_ = [(n, Handle) for n in ("query", "key", "value", "qo_indptr", "kv_indptr",
                                      "output", "lse", "workspace")]


class RopeAppendPlanInfo(C.Structure):
    _fields_ = [("tokens", u64), ("batch_size", u64), ("num_query_heads", u64),
                ("num_kv_heads", u64), ("explicit_tokens", i32), ("workspace_bytes", u64),
                ("validate_blocks", u32)]


class RopeAppendArgs(C.Structure):
    _fields_ = [(n, Handle) for n in ("query", "key", "value", "batch_indices", "positions",
                                      "page_indptr", "page_indices", "last_page_len",
                                      "query_output", "key_pages", "value_pages", "workspace",
                                      "kv_scales")]


class Bf16RopePagedKvAppendArgs(C.Structure):
    _fields_ = [(n, Handle) for n in ("query", "key", "value", "page_indptr", "page_indices",
                                      "last_page_len", "query_output", "key_pages",
                                      "value_pages")]


class Bf16RopePagedKvAppendTokensArgs(C.Structure):
    _fields_ = [(n, Handle) for n in ("query", "key", "value", "batch_indices", "positions",
                                      "page_indptr", "page_indices", "last_page_len",
                                      "query_output", "key_pages", "value_pages")]


P = C.POINTER
pi32 = P(i32)
E = P(Error)

# name -> (restype, argtypes)
SIGNATURES = {
    "loom_abi_version": (u32, []),
    "loom_status_name": (C.c_char_p, [i32]),
    "loom_paged_decode_spec_new": (i32, [u64] * 6 + [P(PagedDecodeSpec), E]),
    "loom_paged_decode_spec_with_page_size": (
        i32, [P(PagedDecodeSpec), u32, P(PagedDecodeSpec), E]),
    "loom_paged_decode_spec_with_kv_dtype": (
        i32, [P(PagedDecodeSpec), u32, P(PagedDecodeSpec), E]),
    "loom_paged_decode_spec_with_kv_layout": (
        i32, [P(PagedDecodeSpec), u32, P(PagedDecodeSpec), E]),
    "loom_paged_prefill_spec_with_page_size": (
        i32, [P(PagedPrefillSpec), u32, P(PagedPrefillSpec), E]),
    "loom_paged_prefill_spec_with_kv_dtype": (
        i32, [P(PagedPrefillSpec), u32, P(PagedPrefillSpec), E]),
    "loom_paged_prefill_spec_with_kv_layout": (
        i32, [P(PagedPrefillSpec), u32, P(PagedPrefillSpec), E]),
    "loom_paged_decode_validate_page_table": (
        i32, [P(PagedDecodeSpec), pi32, u64, pi32, u64, pi32, u64, E]),
    "loom_paged_decode_request_kv_len": (i32, [P(PagedDecodeSpec), pi32, pi32, u64, P(u64)]),
    "loom_paged_decode_physical_page_for_token": (
        i32, [P(PagedDecodeSpec), pi32, pi32, pi32, u64, u64, P(u64), P(u64)]),
    "loom_rope_append_spec_new": (i32, [u64] * 6 + [P(RopeAppendSpec), E]),
    "loom_rope_append_validate_page_table": (
        i32, [P(RopeAppendSpec), pi32, u64, pi32, u64, pi32, u64, E]),
    "loom_rope_append_tokens_spec_new": (i32, [u64] * 7 + [P(RopeAppendTokensSpec), E]),
    "loom_rope_append_tokens_spec_new_extended": (i32, [u64] * 7 + [P(RopeAppendTokensSpec), E]),
    "loom_rope_append_tokens_validate_metadata": (
        i32, [P(RopeAppendTokensSpec), pi32, u64, pi32, u64, pi32, u64, pi32, u64, pi32, u64,
              P(u64), E]),
    "loom_command_queue_new": (i32, [vp, u64, P(vp), E]),
    "loom_command_queue_free": (None, [vp]),
    "loom_command_queue_max_commands": (u64, [vp]),
    "loom_command_queue_reserve_workspace": (i32, [vp, u64, u64, E]),
    "loom_command_queue_workspace_bytes": (u64, [vp]),
    "loom_command_queue_is_poisoned": (C.c_int, [vp]),
    "loom_command_queue_bindings": (i32, [vp, u64, P(vp), E]),
    "loom_bindings_free": (None, [vp]),
    "loom_bindings_len": (u64, [vp]),
    "loom_bindings_capacity": (u64, [vp]),
    "loom_bindings_bind_read": (i32, [vp, vp, u64, C.c_int, P(Handle), E]),
    "loom_bindings_bind_read_write": (i32, [vp, vp, u64, C.c_int, P(Handle), E]),
    "loom_bindings_take_read_write": (i32, [vp, Handle, P(vp), P(u64), E]),
    "loom_command_queue_begin": (i32, [vp, vp, P(vp), E]),
    "loom_command_scope_finish": (i32, [vp, P(vp), E]),
    "loom_command_scope_free": (None, [vp]),
    "loom_command_scope_submitted": (u64, [vp]),
    "loom_command_completion_submitted": (u64, [vp]),
    "loom_command_completion_is_complete": (i32, [vp, P(C.c_int), E]),
    "loom_command_completion_wait": (i32, [vp, P(vp), E]),
    "loom_command_completion_free": (None, [vp]),
    "loom_decode_provider_load": (i32, [C.c_int, P(vp), E]),
    "loom_decode_provider_free": (None, [vp]),
    "loom_decode_provider_plan_bf16_paged_batch": (
        i32, [vp, P(PagedDecodeSpec), P(PagedDecodePlanOptions), P(vp), E]),
    "loom_paged_decode_plan_free": (None, [vp]),
    "loom_paged_decode_plan_get_info": (None, [vp, P(PagedDecodePlanInfo)]),
    "loom_paged_decode_enqueue": (i32, [vp, vp, P(PagedDecodeArgs), E]),
    "loom_paged_decode_enqueue_bf16": (i32, [vp, vp, P(Bf16PagedBatchDecodeArgs), E]),
    "loom_paged_decode_enqueue_bf16_no_alloc": (i32, [vp, vp, P(Bf16PagedBatchDecodeArgs), E]),
    "loom_single_decode_spec_new": (i32, [u64] * 4 + [P(SingleDecodeSpec), E]),
    "loom_single_decode_split_k_spec_new": (
        i32, [P(SingleDecodeSpec), u64, P(SingleDecodeSplitKSpec), E]),
    "loom_single_decode_split_k_partition_token_range": (
        i32, [P(SingleDecodeSplitKSpec), u64, P(u64), P(u64)]),
    "loom_decode_provider_plan_bf16": (i32, [vp, P(SingleDecodeSpec), P(vp), E]),
    "loom_single_decode_plan_free": (None, [vp]),
    "loom_single_decode_enqueue": (i32, [vp, vp, P(SingleDecodeArgs), E]),
    "loom_decode_provider_plan_bf16_split_k": (i32, [vp, P(SingleDecodeSplitKSpec), P(vp), E]),
    "loom_single_decode_split_k_plan_free": (None, [vp]),
    "loom_single_decode_split_k_workspace_bytes": (u64, [vp]),
    "loom_single_decode_split_k_enqueue": (i32, [vp, vp, P(SingleDecodeSplitKArgs), E]),
    "loom_paged_prefill_spec_new": (i32, [u64] * 7 + [P(PagedPrefillSpec), E]),
    "loom_paged_prefill_validate_metadata": (
        i32, [P(PagedPrefillSpec), pi32, u64, pi32, u64, pi32, u64, pi32, u64, E]),
    "loom_paged_prefill_causal_kv_end": (
        i32, [P(PagedPrefillSpec), pi32, pi32, pi32, u64, u64, P(u64)]),
    "loom_prefill_provider_load": (i32, [C.c_int, P(vp), E]),
    "loom_prefill_provider_free": (None, [vp]),
    "loom_prefill_provider_plan_bf16_paged": (i32, [vp, P(PagedPrefillSpec), P(vp), E]),
    "loom_prefill_provider_plan_bf16_paged_options": (
        i32, [vp, P(PagedPrefillSpec), P(PagedPrefillPlanOptions), P(vp), E]),
    "loom_paged_prefill_plan_free": (None, [vp]),
    "loom_paged_prefill_plan_get_info": (None, [vp, P(PagedPrefillPlanInfo)]),
    "loom_paged_prefill_enqueue": (i32, [vp, vp, P(PagedPrefillArgs), E]),
    "loom_ragged_prefill_spec_new": (i32, [u64] * 6 + [P(RaggedPrefillSpec), E]),
    "loom_ragged_prefill_validate_metadata": (i32, [P(RaggedPrefillSpec), pi32, u64, pi32, u64, E]),
    "loom_ragged_prefill_causal_kv_end": (i32, [P(RaggedPrefillSpec), pi32, pi32, u64, u64, P(u64)]),
    "loom_prefill_provider_plan_bf16_ragged": (
        i32, [vp, P(RaggedPrefillSpec), P(PagedPrefillPlanOptions), P(vp), E]),
    "loom_ragged_prefill_plan_free": (None, [vp]),
    "loom_ragged_prefill_plan_get_info": (None, [vp, P(RaggedPrefillPlanInfo)]),
    "loom_ragged_prefill_workspace_numel": (u64, [vp]),
    "loom_ragged_prefill_enqueue": (i32, [vp, vp, P(RaggedPrefillArgs), E]),
    "loom_rope_provider_load": (i32, [C.c_int, P(vp), E]),
    "loom_rope_provider_free": (None, [vp]),
    "loom_rope_provider_plan_bf16_paged_append": (i32, [vp, P(RopeAppendSpec), P(vp), E]),
    "loom_rope_provider_plan_bf16_paged_append_tokens": (
        i32, [vp, P(RopeAppendTokensSpec), P(vp), E]),
    "loom_rope_provider_plan_bf16_paged_append_flags": (
        i32, [vp, P(RopeAppendSpec), u32, P(vp), E]),
    "loom_rope_provider_plan_bf16_paged_append_tokens_flags": (
        i32, [vp, P(RopeAppendTokensSpec), u32, P(vp), E]),
    "loom_rope_append_plan_free": (None, [vp]),
    "loom_rope_append_plan_get_info": (None, [vp, P(RopeAppendPlanInfo)]),
    "loom_rope_append_enqueue": (i32, [vp, vp, P(RopeAppendArgs), E]),
    "loom_rope_append_enqueue_bf16": (i32, [vp, vp, P(Bf16RopePagedKvAppendArgs), E]),
    "loom_rope_append_tokens_enqueue_bf16": (
        i32, [vp, vp, P(Bf16RopePagedKvAppendTokensArgs), E]),
    "loom_graph_queue_new": (i32, [C.c_int, u64, P(vp), E]),
    "loom_graph_queue_free": (None, [vp]),
    "loom_graph_queue_bindings": (i32, [vp, u64, P(vp), E]),
    "loom_graph_queue_reserve_workspace": (i32, [vp, u64, u64, E]),
    "loom_graph_queue_workspace_bytes": (u64, [vp]),
    "loom_graph_queue_begin_capture": (i32, [vp, vp, P(vp), E]),
    "loom_graph_queue_end_capture": (i32, [vp, vp, P(vp), E]),
    "loom_captured_graph_commands": (u64, [vp]),
    "loom_captured_graph_free": (None, [vp]),
    "loom_captured_graph_instantiate": (i32, [vp, P(vp), E]),
    "loom_graph_exec_commands": (u64, [vp]),
    "loom_graph_exec_replay_mode": (i32, [vp]),
    "loom_graph_exec_set_replay_mode": (i32, [vp, i32, E]),
    "loom_graph_exec_launches": (u64, [vp]),
    "loom_graph_exec_launch": (i32, [vp, P(vp), E]),
    "loom_graph_exec_measure_launch_ms": (i32, [vp, vp, vp, P(f32), E]),
    "loom_graph_exec_into_bindings": (i32, [vp, P(vp), E]),
    "loom_graph_exec_free": (None, [vp]),
    "loom_graph_completion_launch_index": (u64, [vp]),
    "loom_graph_completion_is_complete": (i32, [vp, P(C.c_int), E]),
    "loom_graph_completion_wait": (i32, [vp, E]),
    "loom_graph_completion_free": (None, [vp]),
}

_lib = None


def load(path: str = LIB_PATH):
    """Loads the HIP library; raises if it has not been built (no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise RuntimeError(
                f"libloom_infer_hip.so is not built at {path}; run "
                "loom-kernels_amd/build_lib.sh (or __graft_entry__.build())")
        lib = C.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib
