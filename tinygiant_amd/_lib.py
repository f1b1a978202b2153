"""ctypes loader for libtinygiant_hip.so.

Mirrors tinygiant/_lib.py (find_library + load_tinygiant_lib, the same 21
argtype registrations at tinygiant/_lib.py:39-93) and adds the tg_hip_*
device-resident extensions declared in include/tinygiant_hip.h.  The loader
raises if the library is missing: there is no CPU fallback.
"""

import ctypes
from pathlib import Path

VP = ctypes.c_void_p
CI = ctypes.c_int
CF = ctypes.c_float
SZ = ctypes.c_size_t
U64 = ctypes.c_uint64

PKG_DIR = Path(__file__).resolve().parent
LIB_NAME = "libtinygiant_hip.so"


def find_library():
    """Path of the in-tree libtinygiant_hip.so (or its libtinygiant.so alias)."""
    for p in (PKG_DIR / LIB_NAME, PKG_DIR / "libtinygiant.so"):
        if p.exists():
            return p
    return None


def _reg(fn, args, res=None):
    fn.restype = res
    fn.argtypes = args


def register_reference_abi(lib):
    """The reference's own registrations (tinygiant/_lib.py:39-93)."""
    _reg(lib.tg_expert_forward, [VP, VP, VP, CF, CI, CI])
    _reg(lib.tg_expert_forward_mixed, [VP, VP, VP, CI, VP, VP, CF, CI, CI])
    _reg(lib.tg_matmul_q4k, [VP, VP, VP, CI, CI])
    _reg(lib.tg_matmul_q6k, [VP, VP, VP, CI, CI])
    _reg(lib.tg_rms_norm, [VP, VP, VP, CI, CF])
    _reg(lib.tg_f32_matvec, [VP, VP, VP, CI, CI])
    _reg(lib.tg_f16_matvec, [VP, VP, VP, CI, CI])
    _reg(lib.tg_attention_decode,
         [VP, VP, VP, VP, VP, VP, VP, VP, CI, CI, VP, VP, VP, VP, CI, CI, CI, CI, CI])
    _reg(lib.tg_attention_decode_q4,
         [VP, VP, VP, VP, VP, VP, VP, VP, CI, CI, VP, VP, VP, VP, CI, CI, CI, CI, CI])
    _reg(lib.tg_prefetch, [VP, SZ])
    _reg(lib.tg_prefetch_batch, [VP, VP, CI])
    _reg(lib.tg_mlock, [VP, SZ], CI)
    _reg(lib.tg_attention_v2,
         [CI, CI, CI, CI, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP,
          VP, VP, CI, CI, CI, VP, VP, VP, VP, CI, CI, CI, CI, CI, CF])
    _reg(lib.tg_moe_forward_rows_v2,
         [VP, VP, VP, CI, VP, VP, VP, VP, CI, CI, VP, VP, VP, CI, CI, CI])
    _reg(lib.tg_matmul, [CI, VP, VP, VP, VP, CI, CI])
    _reg(lib.tg_row_bytes, [CI, CI], SZ)
    _reg(lib.tg_set_threads, [CI])
    _reg(lib.tg_get_threads, [], CI)
    _reg(lib.tg_expert_forward_rows, [VP, VP, VP, CI, VP, VP, VP, CI, CI, CI])
    _reg(lib.tg_moe_forward_rows, [VP, VP, VP, VP, CI, VP, VP, VP, CI, CI, CI])
    _reg(lib.tg_transformer_layer,
         [VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, CI, CI, VP, VP,
          VP, VP, VP, VP, VP, CI, VP, CI, CI, CI, CI, CI, CI])


def register_extensions(lib):
    """tg_hip_* entry points (include/tinygiant_hip.h, part 2)."""
    _reg(lib.tg_moe_forward, [VP, VP, CI, VP, VP, CI, CI])
    _reg(lib.tg_hip_last_error, [], ctypes.c_char_p)
    _reg(lib.tg_hip_clear_error, [])
    _reg(lib.tg_hip_register, [VP, SZ], CI)
    _reg(lib.tg_hip_unregister, [VP], CI)
    _reg(lib.tg_hip_registered_bytes, [], SZ)
    _reg(lib.tg_hip_device_ptr, [VP, SZ], VP)
    _reg(lib.tg_hip_stream, [], VP)
    _reg(lib.tg_hip_malloc, [SZ], VP)
    _reg(lib.tg_hip_free, [VP])
    _reg(lib.tg_hip_memcpy_h2d, [VP, VP, SZ])
    _reg(lib.tg_hip_memcpy_d2h, [VP, VP, SZ])
    _reg(lib.tg_hip_memcpy_d2d, [VP, VP, SZ, VP])
    _reg(lib.tg_hip_synchronize, [])
    _reg(lib.tg_hip_shutdown, [])
    _reg(lib.tg_hip_synth_fill, [CI, U64, VP, U64, VP])
    _reg(lib.tg_hip_synth_fill_host, [CI, U64, VP, U64])
    _reg(lib.tg_hip_quantize_q8, [VP, CI, CI, VP])
    _reg(lib.tg_hip_isums, [CI, VP, CI, CI, VP, VP], CI)
    _reg(lib.tg_hip_moe_plan_create,
         [VP, VP, VP, CI, VP, VP, VP, VP, CI, CI, VP, CI, CI, CI], VP)
    _reg(lib.tg_hip_moe_plan_run, [VP, VP, VP, VP])
    _reg(lib.tg_hip_moe_plan_pairs, [VP], CI)
    _reg(lib.tg_hip_moe_plan_destroy, [VP])
    _reg(lib.tg_hip_matmul_dev, [CI, VP, VP, VP, VP, CI, CI, CI, VP, VP])
    _reg(lib.tg_hip_matmul_scratch_bytes, [CI, CI], SZ)
    _reg(lib.tg_hip_init, [])
    _reg(lib.tg_hip_matmul_dev_noalloc, [CI, VP, VP, VP, VP, CI, CI, CI, VP])
    _reg(lib.tg_hip_matmul_noalloc_max_bytes, [], SZ)
    _reg(lib.tg_hip_head_argmax_dev, [CI, VP, VP, VP, CF, CI, CI, CI, VP, VP, VP, VP, VP])
    _reg(lib.tg_hip_head_scratch_bytes, [CI, CI, CI], SZ)
    _reg(lib.tg_hip_route_dev, [VP, VP, VP, CI, CI, CI, CI, VP, VP, VP, VP])
    _reg(lib.tg_hip_route_scratch_bytes, [CI, CI], SZ)
    _reg(lib.tg_hip_route_restricted_dev, [VP, VP, VP, CI, CI, CI, CI, VP, VP, VP, VP, VP])
    _reg(lib.tg_hip_attention_dev, [CI, CI, CI, CI, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, CI, CI, CI,
                                    VP, VP, VP, VP, CI, CI, CI, CI, CI, CF, VP, VP, VP])
    _reg(lib.tg_hip_attention_scratch_bytes, [CI, CI, CI, CI, CI], SZ)
    _reg(lib.tg_hip_upload_file, [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_uint64, VP, ctypes.c_uint64],
         ctypes.c_int64)
    _reg(lib.tg_hip_mark, [CI])
    _reg(lib.tg_hip_set_moe_grouped_min_rows, [CI], CI)
    _reg(lib.tg_hip_set_moe_qk_min_rows, [CI], CI)
    _reg(lib.tg_hip_set_head_mfma_min_k, [CI], CI)
    _reg(lib.tg_hip_set_moe_expert_major, [CI], CI)
    _reg(lib.tg_hip_marks_ms, [CI, CI], CF)
    _reg(lib.tg_hip_rms_norm_dev, [VP, VP, VP, CI, CI, CF, VP])
    _reg(lib.tg_hip_moe_forward_stages,
         [VP, VP, VP, CI, VP, VP, VP, VP, CI, CI, VP, VP, VP, CI, CI, CI, VP, VP])
    _reg(lib.tg_hip_decode_create, [VP, CI, VP, CF, VP, CI], VP)
    _reg(lib.tg_hip_decode_run, [VP, VP])
    _reg(lib.tg_hip_decode_time, [VP, CI], CF)
    _reg(lib.tg_hip_decode_kernel_times, [VP, VP, VP])
    _reg(lib.tg_hip_decode_destroy, [VP])
    _reg(lib.tg_hip_decode_status, [VP], CI)
    _reg(lib.tg_hip_decode_set_policy, [VP, CI], CI)
    _reg(lib.tg_hip_decode_placement, [VP, VP], CI)
    _reg(lib.tg_hip_decode_set_debug, [VP, VP])
    _reg(lib.tg_hip_decode_debug_bytes, [], SZ)
    _reg(lib.tg_hip_decode_record_bytes, [VP], SZ)
    _reg(lib.tg_hip_decode_set_timing, [VP, VP])
    _reg(lib.tg_hip_device_name, [ctypes.c_char_p, CI])
    _reg(lib.tg_hip_copy_time, [VP, VP, U64, CI], CF)


def load_tinygiant_lib(lib_path=None):
    """Loads libtinygiant_hip.so with every registration.  Unlike the
    reference (which returns None when nothing is found), a missing library
    is an error: the hot path has no fallback."""
    if lib_path is None:
        lib_path = find_library()
    if lib_path is None:
        raise RuntimeError(
            f"{LIB_NAME} is not built in {PKG_DIR}; run `python -m tinygiant_amd.build` "
            "(or __graft_entry__.build()) first")
    lib = ctypes.CDLL(str(lib_path))
    register_reference_abi(lib)
    register_extensions(lib)
    return lib
