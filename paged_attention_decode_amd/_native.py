"""Loaders for the in-tree native libraries (no CPU fallback).

* ``ext()`` - the PyTorch binding ``_pa_decode_ext`` (pa_torch.cpp), which
  calls the C ABI.  Importing it needs ``torch`` already imported (it links
  against PyTorch's HIP runtime).
* ``capi()`` - ``libpa_decode.so`` opened with ctypes, with argument types
  for every entry point of include/pa_decode.h, plus the ``PadDims`` /
  ``PadPlan`` / ``PadCall`` structures that mirror ``pad_decode_dims`` /
  ``pad_decode_plan_t`` / ``pad_decode_call``.
* ``probe()`` - ``libpa_probe.so``, the bandwidth probes used by
  ``roofline.py`` (measurement tooling, not the decode path).
* ``timeline()`` - ``libpa_decode_tl.so``, the decode library built with
  per-workgroup phase stamps (include/pa_decode_timeline.h), for
  ``profile_run --timeline`` (measurement tooling, not the decode path).

Both raise ImportError with the build command when the library is missing;
nothing here computes attention on the CPU.
"""

from __future__ import annotations

import ctypes
import importlib.util
import os
import sysconfig

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CAPI_PATH = os.path.join(_PKG_DIR, "libpa_decode.so")
EXT_PATH = os.path.join(_PKG_DIR, "_pa_decode_ext" + sysconfig.get_config_var("EXT_SUFFIX"))
_BUILD_HINT = "build it with `python -m paged_attention_decode_amd.build` (or __graft_entry__.build())"

_ext = None
_capi = None


def ext():
    """The PyTorch extension module (loaded once)."""
    global _ext
    if _ext is None:
        if not os.path.exists(EXT_PATH):
            raise ImportError(f"paged_attention_decode_amd: {EXT_PATH} is missing; {_BUILD_HINT}")
        import torch  # noqa: F401  (the extension resolves symbols from torch's libraries)

        spec = importlib.util.spec_from_file_location("_pa_decode_ext", EXT_PATH)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _ext = mod
    return _ext


class PadDims(ctypes.Structure):
    """Mirror of ``pad_decode_dims`` (include/pa_decode.h)."""

    _fields_ = [
        ("batch", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("max_pages", ctypes.c_int32),
        ("num_pages", ctypes.c_int64),
        ("q_stride", ctypes.c_int64 * 3),
        ("k_stride", ctypes.c_int64 * 4),
        ("v_stride", ctypes.c_int64 * 4),
        ("bt_stride", ctypes.c_int64 * 2),
        ("sl_stride", ctypes.c_int64),
        ("out_stride", ctypes.c_int64 * 3),
    ]


class PadPlan(ctypes.Structure):
    """Mirror of ``pad_decode_plan_t`` (include/pa_decode.h)."""

    _fields_ = [
        ("num_splits", ctypes.c_int32),
        ("pages_per_split", ctypes.c_int32),
        ("waves_per_group", ctypes.c_int32),
        ("single_pass", ctypes.c_int32),
        ("engine", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("workspace_bytes", ctypes.c_size_t),
        ("counters", ctypes.c_int64),
    ]


class PadCall(ctypes.Structure):
    """Mirror of ``pad_decode_call`` (include/pa_decode.h)."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k_cache", ctypes.c_void_p),
        ("v_cache", ctypes.c_void_p),
        ("block_table", ctypes.c_void_p),
        ("seq_lens", ctypes.c_void_p),
        ("indptr", ctypes.c_void_p),
        ("last_page_len", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("counters", ctypes.c_void_p),
        ("num_counters", ctypes.c_int64),
        ("worklist", ctypes.c_void_p),
        ("worklist_bytes", ctypes.c_size_t),
        ("scale", ctypes.c_float),
        ("num_splits", ctypes.c_int32),
        ("engine", ctypes.c_int32),
        ("kv_format", ctypes.c_int32),
        ("k_scale", ctypes.c_float),
        ("v_scale", ctypes.c_float),
    ]


# Exported entry points and their C signatures (argtypes, restype).
_VP = ctypes.c_void_p
SIGNATURES = {
    "pad_decode_plan": ([ctypes.POINTER(PadDims), ctypes.c_int, ctypes.c_int, ctypes.POINTER(PadPlan)], ctypes.c_int),
    "pad_decode_plan_csr": (
        [ctypes.POINTER(PadDims), ctypes.c_int, ctypes.c_int, ctypes.POINTER(PadPlan)], ctypes.c_int),
    "pad_decode_workspace_bytes": (
        [ctypes.POINTER(PadDims), ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_size_t)],
        ctypes.c_int,
    ),
    "pad_decode_counters_needed": (
        [ctypes.POINTER(PadDims), ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_int64)],
        ctypes.c_int,
    ),
    "pad_decode_counters_init": ([_VP, ctypes.c_int64, _VP], ctypes.c_int),
    "pad_decode_launch": (
        [_VP, _VP, _VP, _VP, _VP, _VP, _VP, ctypes.c_size_t, _VP, ctypes.c_int64, ctypes.POINTER(PadDims),
         ctypes.c_float, ctypes.c_int, _VP],
        ctypes.c_int,
    ),
    "pad_decode_launch_kv8": (
        [_VP, _VP, _VP, _VP, _VP, _VP, _VP, ctypes.c_size_t, _VP, ctypes.c_int64, ctypes.POINTER(PadDims),
         ctypes.c_float, ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_int, _VP],
        ctypes.c_int,
    ),
    "pad_decode_launch_ex": (
        [_VP, _VP, _VP, _VP, _VP, _VP, _VP, ctypes.c_size_t, _VP, ctypes.c_int64, ctypes.POINTER(PadDims),
         ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_VP), _VP],
        ctypes.c_int,
    ),
    "pad_decode_launch_csr": (
        [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, ctypes.c_size_t, _VP, ctypes.c_int64, ctypes.POINTER(PadDims),
         ctypes.c_float, ctypes.c_int, ctypes.c_int, _VP],
        ctypes.c_int,
    ),
    "pad_decode_launch_noalloc": (
        [_VP, _VP, _VP, _VP, _VP, _VP, ctypes.POINTER(PadDims), ctypes.c_float, ctypes.c_int, _VP], ctypes.c_int),
    "pad_decode_worklist_bytes": (
        [ctypes.POINTER(PadDims), ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_size_t)],
        ctypes.c_int,
    ),
    "pad_decode_plan_worklist": (
        [_VP, _VP, ctypes.POINTER(PadDims), ctypes.c_int, _VP, ctypes.c_size_t, _VP], ctypes.c_int),
    "pad_decode_plan_worklist_csr": (
        [_VP, _VP, _VP, ctypes.POINTER(PadDims), ctypes.c_int, _VP, ctypes.c_size_t, _VP], ctypes.c_int),
    "pad_decode_launch_worklist": (
        [_VP, _VP, _VP, _VP, _VP, _VP, _VP, ctypes.c_size_t, _VP, ctypes.c_int64, ctypes.POINTER(PadDims),
         ctypes.c_float, ctypes.c_int, _VP, ctypes.c_size_t, _VP],
        ctypes.c_int,
    ),
    "pad_decode_launch_worklist_csr": (
        [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, ctypes.c_size_t, _VP, ctypes.c_int64, ctypes.POINTER(PadDims),
         ctypes.c_float, ctypes.c_int, _VP, ctypes.c_size_t, _VP],
        ctypes.c_int,
    ),
    "pad_decode_launch_call": ([ctypes.POINTER(PadCall), ctypes.POINTER(PadDims), _VP], ctypes.c_int),
    "pad_decode_plan_worklist_call": (
        [ctypes.POINTER(PadCall), ctypes.POINTER(PadDims), _VP, ctypes.c_size_t, _VP], ctypes.c_int),
    "pad_device_num_cus": ([ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
    "pad_status_string": ([ctypes.c_int], ctypes.c_char_p),
    "pad_decode_abi_version": ([], ctypes.c_int),
}


def capi():
    """ctypes handle to libpa_decode.so with typed entry points (loaded once)."""
    global _capi
    if _capi is None:
        if not os.path.exists(CAPI_PATH):
            raise ImportError(f"paged_attention_decode_amd: {CAPI_PATH} is missing; {_BUILD_HINT}")
        lib = ctypes.CDLL(CAPI_PATH)
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _capi = lib
    return _capi


TIMELINE_PATH = os.path.join(_PKG_DIR, "libpa_decode_tl.so")
TIMELINE_SIGNATURES = {
    "pad_timeline_read": ([_VP, ctypes.c_size_t], ctypes.c_int),
    "pad_timeline_reset": ([], ctypes.c_int),
}
# include/pa_decode_timeline.h
TL_LAUNCHES, TL_MAX_GROUPS, TL_SLOTS = 4, 16384, 8
TL_ENTRY, TL_ITEM, TL_LOOP_END, TL_PUBLISHED, TL_ARRIVED, TL_MERGED, TL_EXIT, TL_INFO = range(8)
TL_F_NO_ITEM, TL_F_SINGLE, TL_F_MERGER, TL_F_GROUP = 1, 2, 4, 8
_timeline = None


def timeline():
    """ctypes handle to libpa_decode_tl.so: every decode entry point plus the stamp buffer readers."""
    global _timeline
    if _timeline is None:
        if not os.path.exists(TIMELINE_PATH):
            raise ImportError(f"paged_attention_decode_amd: {TIMELINE_PATH} is missing; {_BUILD_HINT}")
        lib = ctypes.CDLL(TIMELINE_PATH)
        for name, (argtypes, restype) in {**SIGNATURES, **TIMELINE_SIGNATURES}.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _timeline = lib
    return _timeline


PROBE_PATH = os.path.join(_PKG_DIR, "libpa_probe.so")
PROBE_SIGNATURES = {
    "pad_probe_stream_read": (
        [_VP, ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int, _VP, _VP],
        ctypes.c_int,
    ),
    "pad_probe_paged_read": (
        [_VP, _VP, _VP, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
         ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, _VP, _VP],
        ctypes.c_int,
    ),
}
_probe = None


def probe():
    """ctypes handle to libpa_probe.so (bandwidth probes of the roofline report)."""
    global _probe
    if _probe is None:
        if not os.path.exists(PROBE_PATH):
            raise ImportError(f"paged_attention_decode_amd: {PROBE_PATH} is missing; {_BUILD_HINT}")
        lib = ctypes.CDLL(PROBE_PATH)
        for name, (argtypes, restype) in PROBE_SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _probe = lib
    return _probe


def dims_for(q, k_cache, v_cache, block_table, seq_lens, out) -> PadDims:
    """Fill a PadDims from tensors (shapes + element strides)."""
    d = PadDims()
    d.batch, d.num_q_heads, d.head_dim = (int(x) for x in q.shape)
    d.num_pages, d.page_size, d.num_kv_heads = int(k_cache.shape[0]), int(k_cache.shape[1]), int(k_cache.shape[2])
    d.max_pages = int(block_table.shape[1])
    for i in range(3):
        d.q_stride[i] = q.stride(i)
        d.out_stride[i] = out.stride(i)
    for i in range(4):
        d.k_stride[i] = k_cache.stride(i)
        d.v_stride[i] = v_cache.stride(i)
    d.bt_stride[0], d.bt_stride[1] = block_table.stride(0), block_table.stride(1)
    d.sl_stride = seq_lens.stride(0)
    return d
