"""Loader for the gfx950 hot-tier library (libhotcold_hip.so, C ABI in
include/hotcold_hip.h).

The library is the only compute path of this package: if it is missing or the
tensors are not on a ROCm device, the ops raise instead of falling back to
another implementation.
"""

import ctypes
import os
import threading

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libhotcold_hip.so")
_lock = threading.Lock()
_lib = None

HC_OK = 0
HC_ERR_INVALID = -1
HC_ERR_HIP = -2
HC_ERR_UNSUPPORTED = -3
HC_ERR_WORKSPACE = -4
HC_ERR_GROUP = -5
HC_ERR_DROPOUT = -6

HC_DTYPE_F32 = 0
HC_DTYPE_F16 = 1
HC_DTYPE_BF16 = 2

HC_POOL_MAX = 0
HC_POOL_AVG = 1

HC_SCORE_SNAPKV = 0
HC_SCORE_RAWSUM = 1

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p
_dbl = ctypes.c_double

# name -> (restype, argtypes)
SIGNATURES = {
    "hc_abi_version": (_int, []),
    "hc_last_error": (ctypes.c_char_p, []),
    "hc_read_bytes": (_int, [_vp, _i64, _vp, _vp]),
    "hc_decode_attn_workspace_size": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64, _int]),
    "hc_decode_attn": (_int, [
        _int, _i64, _i64, _i64, _i64, _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64,
        _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64,
        _vp,
        _dbl, _dbl,
        _vp, _i64, _i64,
        _vp, _vp,
        _vp, _i64, _i64,
        _vp]),
    "hc_decode_attn_append": (_int, [
        _int, _i64, _i64, _i64, _i64, _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _vp, _i64,
        _vp, _i64,
        _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64,
        _vp,
        _dbl,
        _vp, _i64, _i64,
        _vp, _i64, _i64,
        _vp]),
    "hc_decode_attn_append_packed": (_int, [_vp, _vp]),
    "hc_decode_append_args_size": (_i64, []),
    "hc_decode_attn_h2o_evict_packed": (_int, [_vp, _vp]),
    "hc_decode_h2o_evict_args_size": (_i64, []),
    "hc_decode_attn_append_noalloc": (_int, [
        _int, _i64, _i64, _i64, _i64, _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _vp, _i64,
        _vp, _i64,
        _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64,
        _vp,
        _dbl,
        _vp, _i64, _i64,
        _i64,
        _vp]),
    "hc_decode_attn_h2o": (_int, [
        _int, _i64, _i64, _i64, _i64, _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _dbl,
        _vp, _i64, _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64, _vp]),
    "hc_decode_attn_h2o_evict": (_int, [
        _int, _i64, _i64, _i64, _i64, _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64,
        _dbl,
        _vp, _i64, _i64,
        _vp, _i64, _i64,
        _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64,
        _vp, _i64, _i64, _vp]),
    "hc_snapkv_score_workspace_size": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "hc_snapkv_score": (_int, [
        _int, _int, _i64, _i64, _i64, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _dbl, _i64, _int,
        _vp,
        _vp, _i64, _vp]),
    "hc_snapkv_score_rows": (_int, [
        _int, _int, _i64, _i64, _i64, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64,
        _dbl, _i64, _int,
        _vp,
        _vp, _i64, _vp]),
    "hc_head_mean": (_int, [_i64, _i64, _i64, _vp, _vp, _vp]),
    "hc_topk_keep": (_int, [_i64, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp]),
    "hc_topk_keep_workspace_size": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "hc_topk_keep_ws": (_int, [_i64, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp]),
    "hc_gather_rows": (_int, [
        _i64, _i64, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64,
        _vp, _i64, _vp, _i64,
        _vp]),
    "hc_gather_rows_tab": (_int, [
        _i64, _i64, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64, _i64,
        _vp, _i64, _i64, _vp, _i64, _i64,
        _vp, _i64, _i64, _vp, _i64, _i64,
        _vp]),
    "hc_append_rows": (_int, [
        _int, _i64, _i64, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64,
        _vp, _i64, _vp, _i64,
        _vp]),
    "hc_inject_rerope": (_int, [
        _int, _i64, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64,
        _vp, _dbl,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp]),
    "hc_inject_rerope_tab": (_int, [
        _int, _i64, _i64, _i64, _i64, _int,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp]),
    "hc_stream_create": (_int, [ctypes.POINTER(_vp)]),
    "hc_stream_destroy": (_int, [_vp]),
    "hc_event_create": (_int, [ctypes.POINTER(_vp), _int]),
    "hc_event_destroy": (_int, [_vp]),
    "hc_event_record": (_int, [_vp, _vp]),
    "hc_event_query": (_int, [_vp]),
    "hc_event_synchronize": (_int, [_vp]),
    "hc_event_elapsed_ms": (_int, [_vp, _vp, ctypes.POINTER(ctypes.c_float)]),
    "hc_stream_wait_event": (_int, [_vp, _vp]),
    "hc_memcpy_h2d_async": (_int, [_vp, _vp, _i64, _vp]),
    "hc_memcpy_d2h_async": (_int, [_vp, _vp, _i64, _vp]),
    "hc_gather_evict_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "hc_gather_evict": (_int, [_int, _i64, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64,
                               _vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _vp]),
    # host cold store
    "hc_cold_create": (_vp, [_i64, _i64, _i64, _i64, _i64, _int]),
    "hc_cold_destroy": (None, [_vp]),
    "hc_cold_size": (_i64, [_vp]),
    "hc_cold_add": (_int, [_vp, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp]),
    "hc_cold_search": (_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "hc_cold_export": (_int, [_vp, _vp, _vp, _vp, _vp]),
    "hc_cold_retrieve": (_int, [_vp, _i64, _vp, _i64, _i64, _i64, _int, _i64, _int, _int, _vp, _vp, _vp, _vp,
                                _vp, _i64, _i64, _vp, _vp, _i64]),
    "hc_cold_retrieve_async": (_vp, [_vp, _i64, _vp, _i64, _i64, _i64, _int, _i64, _int, _int, _vp, _vp, _vp, _vp,
                                     _vp, _i64, _i64, _vp, _i64, _vp, _i64]),
    "hc_cold_add_async": (_vp, [_vp, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _i64]),
    "hc_cold_defer_vectors": (_int, [_vp, _int]),
    "hc_cold_gather": (_int, [_vp, _i64, _int, _i64, _vp, _int, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _vp,
                              _i64]),
    "hc_cold_gather_async": (_vp, [_vp, _i64, _int, _i64, _vp, _int, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64,
                                   _vp, _i64]),
    "hc_cold_job_poll": (_int, [_vp, _int, _vp, _vp]),
    "hc_cold_job_free": (None, [_vp]),
    "hc_index_add": (_int, [_i64, _i64, _i64, _i64, _i64, _int, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i64,
                             _vp]),
    "hc_index_search": (_int, [_i64, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _int, _vp, _vp, _int, _i64, _vp, _vp,
                                _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "hc_retrieval_query_max_rows": (_i64, []),
    "hc_retrieval_query": (_int, [_int, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _int, _vp, _vp, _vp, _vp]),
}


class DecodeAppendArgs(ctypes.Structure):
    """ctypes mirror of hc_decode_append_args (include/hotcold_hip.h): every
    field 8 bytes, in the header's order."""
    _fields_ = [(n, t) for names, t in (
        ("dtype B Hq Hk D S", _i64), ("q", _vp), ("q_sb q_sh", _i64), ("k", _vp), ("k_sb k_sh k_ss", _i64),
        ("v", _vp), ("v_sb v_sh v_ss", _i64), ("k_new", _vp), ("kn_sb kn_sh", _i64), ("v_new", _vp),
        ("vn_sb vn_sh", _i64), ("p_new", _vp), ("pn_sb pn_sh", _i64), ("p_dst", _vp), ("pd_sb pd_sh pd_ss", _i64),
        ("pos_new", _vp), ("posn_sb", _i64), ("pos_dst", _vp), ("posd_sb", _i64), ("mask", _vp), ("mask_sb", _i64),
        ("held_len", _i64), ("held_pos", _vp), ("hp_sb hp_sh", _i64), ("held_valid", _vp), ("hv_sb hv_sh", _i64),
        ("cur_pos", _vp), ("scaling", _dbl), ("out", _vp), ("o_sb o_sh", _i64), ("workspace", _vp),
        ("workspace_bytes num_splits", _i64)) for n in names.split()]


class DecodeH2OEvictArgs(ctypes.Structure):
    """ctypes mirror of hc_decode_h2o_evict_args (include/hotcold_hip.h):
    every field 8 bytes, in the header's order."""
    _fields_ = [(n, t) for names, t in (
        ("dtype B Hq Hk D S", _i64), ("q", _vp), ("q_sb q_sh", _i64), ("k", _vp), ("k_sb k_sh k_ss", _i64),
        ("v", _vp), ("v_sb v_sh v_ss", _i64), ("k_new", _vp), ("kn_sb kn_sh", _i64), ("v_new", _vp),
        ("vn_sb vn_sh", _i64), ("scaling", _dbl), ("out", _vp), ("o_sb o_sh", _i64), ("acc", _vp),
        ("a_sb a_sh window budget", _i64), ("k_dst", _vp), ("kd_sb kd_sh kd_ss", _i64), ("v_dst", _vp),
        ("vd_sb vd_sh vd_ss", _i64), ("acc_dst", _vp), ("ad_sb ad_sh", _i64), ("workspace", _vp),
        ("workspace_bytes num_splits", _i64)) for n in names.split()]


def library_path():
    return _LIB_PATH


def lib():
    """Return the loaded library, loading it on first use; raise if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(
                f"hotcold_kv: native library not built ({_LIB_PATH}); "
                "run `python hotcold-kv-cache_amd/build_native.py`")
        handle = ctypes.CDLL(_LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.hc_decode_append_args_size() != ctypes.sizeof(DecodeAppendArgs):
            raise RuntimeError("hotcold_kv: hc_decode_append_args layout differs between the library and the binding")
        if handle.hc_decode_h2o_evict_args_size() != ctypes.sizeof(DecodeH2OEvictArgs):
            raise RuntimeError("hotcold_kv: hc_decode_h2o_evict_args layout differs between the library and the binding")
        _lib = handle
    return _lib


_BIND_PATH = os.path.join(os.path.dirname(_LIB_PATH), "hc_step_bind.so")
_bind = None
_bind_tried = False


def step_bind():
    """The decode loop's native per-step call (csrc/bind/hc_step_bind.cpp, a
    Python extension module beside the library), or None where it is not
    built: the packed decode call then marshals its step from Python through
    ctypes, into the same library and kernels."""
    global _bind, _bind_tried
    if _bind_tried:
        return _bind
    if os.path.exists(_BIND_PATH):
        lib()                                           # the module links against the library (loads under _lock)
    with _lock:
        if not _bind_tried:
            if os.path.exists(_BIND_PATH):
                import importlib.util
                spec = importlib.util.spec_from_file_location("hc_step_bind", _BIND_PATH)
                mod = importlib.util.module_from_spec(spec)
                spec.loader.exec_module(mod)
                _bind = mod
            _bind_tried = True
    return _bind


class HotColdError(RuntimeError):
    pass


def check(rc, what):
    """Map a C-ABI status to the reference's exception types."""
    if rc == HC_OK:
        return
    msg = lib().hc_last_error().decode(errors="replace")
    if rc in (HC_ERR_GROUP, HC_ERR_DROPOUT):
        raise ValueError(msg)
    raise HotColdError(f"{what}: {msg} (status {rc})")


def dtype_code(dtype):
    if dtype == torch.float16:
        return HC_DTYPE_F16
    if dtype == torch.bfloat16:
        return HC_DTYPE_BF16
    if dtype == torch.float32:
        return HC_DTYPE_F32
    raise TypeError(f"hotcold_kv: unsupported dtype {dtype}")
