"""ctypes view of libfdi4's C ABI (include/fdi4.h).

For callers that hold raw device pointers and no torch binding (the shape a
cgo / JNI / N-API binding of the reference's cu_* functions would take).
Loading the library needs no GPU; calling a compute entry point does.
"""

import ctypes
import os

from ._lib import LIB_PATH

c_int, c_int32, c_int64, c_size_t, c_void_p = (ctypes.c_int, ctypes.c_int32, ctypes.c_int64,
                                                ctypes.c_size_t, ctypes.c_void_p)

V_F32 = 0
V_F16 = 1
V_BF16 = 2
K_F32, K_F16, K_BF16 = 0, 1, 2
ROUND_HALF_UP, ROUND_HALF_EVEN = 0, 1
SCALE_DIVIDE, SCALE_RECIPROCAL = 0, 1
#: FDI4_NOALLOC_SCRATCH_BYTES: the split partials fdi4_decode_paged_noalloc holds.
NOALLOC_SCRATCH_BYTES = 8 << 20
#: fdi4_tuning_knob codes (launch-shape overrides for measurement and tests).
TUNE = {"decode_vector_only": 0, "decode_waves": 1, "decode_heads_per_wg": 2,
        "decode_target_waves": 3, "fake_quant_split": 4}


class PagedCache(ctypes.Structure):
    """Mirror of ``fdi4_paged_cache``."""
    _fields_ = [
        ("k_pages", c_void_p),
        ("k_page_stride", c_int64), ("k_head_stride", c_int64), ("k_row_stride", c_int64),
        ("v_pages", c_void_p),
        ("v_dtype", c_int32),
        ("v_page_stride", c_int64), ("v_head_stride", c_int64), ("v_row_stride", c_int64),
        ("k_scale", c_void_p),
        ("k_zp", c_void_p),
        ("s_batch_stride", c_int64), ("s_head_stride", c_int64),
        ("s_group_stride", c_int64), ("s_page_stride", c_int64),
        ("page_table", c_void_p),
        ("pt_batch_stride", c_int64),
        ("seq_lens", c_void_p),
        ("page_lens", c_void_p),
        ("pl_batch_stride", c_int64),
        ("num_kv_heads", c_int32),
        ("head_dim", c_int32),
        ("page_rows", c_int32),
        ("pages_per_group", c_int32),
        ("max_pages", c_int32),
        ("num_pages", c_int32),
    ]


#: name -> (restype, argtypes); the complete exported surface of include/fdi4.h.
SIGNATURES = {
    "fdi4_set_tuning": (c_int, [c_int, c_int]),
    "fdi4_get_tuning": (c_int, [c_int]),
    "fdi4_abi_version": (c_int, []),
    "fdi4_error_string": (ctypes.c_char_p, [c_int]),
    "fdi4_quantize_int4": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p,
                                   c_void_p]),
    "fdi4_quantize_rows_workspace_bytes": (c_size_t, [c_int64, c_int]),
    "fdi4_quantize_rows": (c_int, [c_void_p, c_int64, c_int, c_int64, c_void_p, c_int64, c_int,
                                   c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "fdi4_quantize_paged": (c_int, [c_void_p, c_int, c_int, c_int64, c_int64, c_int64, c_int,
                                    ctypes.POINTER(PagedCache), c_void_p]),
    "fdi4_append_paged": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_int,
                                  c_void_p, c_int64, c_int64, c_int64, c_int,
                                  ctypes.POINTER(PagedCache), c_void_p]),
    "fdi4_append_paged_advance": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64,
                                          c_int64, c_int, c_void_p, c_int64, c_int64, c_int64,
                                          c_int, ctypes.POINTER(PagedCache), c_void_p,
                                          c_void_p]),
    "fdi4_flash_decode_int4": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p,
                                       c_void_p]),
    "fdi4_flash_decode_int4_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "fdi4_flash_decode_int4_ws": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                          c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p,
                                          c_void_p, c_size_t, c_void_p]),
    "fdi4_decode_num_splits": (c_int, [c_int, c_int, ctypes.POINTER(PagedCache)]),
    "fdi4_decode_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "fdi4_decode_paged": (c_int, [c_void_p, c_int, c_int, c_int64, c_int64,
                                  ctypes.POINTER(PagedCache), c_void_p, c_int64, c_int64, c_int,
                                  c_void_p, c_size_t, c_void_p]),
    "fdi4_decode_paged_ex": (c_int, [c_void_p, c_int, c_int, c_int, c_int64, c_int64,
                                     ctypes.POINTER(PagedCache), c_void_p, c_int, c_int64,
                                     c_int64, c_int, c_void_p, c_size_t, c_void_p]),
    "fdi4_decode_paged_advance": (c_int, [c_void_p, c_int, c_int, c_int, c_int64, c_int64,
                                          ctypes.POINTER(PagedCache), c_void_p, c_int, c_int64,
                                          c_int64, c_int, c_void_p, c_size_t, c_void_p,
                                          c_void_p]),
    "fdi4_decode_step": (c_int, [c_void_p, c_int, c_int, c_int, c_int64, c_int64, c_void_p,
                                 c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int64,
                                 c_int64, c_int64, c_int, ctypes.POINTER(PagedCache), c_void_p,
                                 c_int, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_size_t,
                                 c_void_p]),
    "fdi4_decode_partials_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "fdi4_decode_paged_partials": (c_int, [c_void_p, c_int, c_int, c_int64, c_int64,
                                           ctypes.POINTER(PagedCache), c_int, c_void_p,
                                           c_size_t, c_void_p]),
    "fdi4_decode_paged_noalloc": (c_int, [c_void_p, c_int, c_int, c_int64, c_int64,
                                          ctypes.POINTER(PagedCache), c_void_p, c_int64,
                                          c_int64, c_int, c_void_p]),
    "fdi4_merge_splits": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p,
                                  c_int64, c_int64, c_void_p]),
    "fdi4_dequantize_int4": (c_int, [c_void_p, c_int64, c_int, c_int64, c_int, c_void_p,
                                     c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p]),
    "fdi4_pack_int4": (c_int, [c_void_p, c_int64, c_int, c_int64, c_void_p, c_int64, c_int,
                               c_void_p]),
    "fdi4_fake_quantize": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_int64,
                                   c_int64, c_int64, c_void_p, c_int64, c_int64, c_int64, c_int,
                                   c_int, c_int, c_void_p]),
}

_lib = None


def load(path: str = LIB_PATH):
    """dlopen libfdi4.so and attach the prototypes (no GPU needed)."""
    global _lib
    if _lib is not None and path == LIB_PATH:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run `python -m flash_decode_int4._build`")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path == LIB_PATH:
        _lib = lib
    return lib


def check(rc: int, what: str = "fdi4 call") -> None:
    if rc != 0:
        msg = load().fdi4_error_string(rc)
        raise RuntimeError(f"{what} failed ({rc}): {msg.decode() if msg else ''}")


class tuning:
    """Context manager that sets launch-shape overrides (``fdi4_set_tuning``)
    for the calls made inside it and restores the previous values on exit:

        with capi.tuning(decode_vector_only=1):
            out = ops.flash_decode_paged(...)

    Process-wide: calls made meanwhile on other threads see the settings too.
    """

    def __init__(self, **knobs):
        unknown = set(knobs) - set(TUNE)
        if unknown:
            raise ValueError(f"unknown tuning knobs {sorted(unknown)}; known: {sorted(TUNE)}")
        self._knobs = {TUNE[k]: int(v) for k, v in knobs.items()}
        self._saved = {}

    def __enter__(self):
        lib = load()
        for knob, value in self._knobs.items():
            self._saved[knob] = lib.fdi4_get_tuning(knob)
            check(lib.fdi4_set_tuning(knob, value), f"fdi4_set_tuning({knob}, {value})")
        return self

    def __exit__(self, *exc):
        lib = load()
        for knob, value in self._saved.items():
            lib.fdi4_set_tuning(knob, value)
        return False
