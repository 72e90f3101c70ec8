"""ctypes binding of librk_path.so, the HIP C ABI declared in include/rk_path.h.

The counterpart of the reference's src/native/metal_native.py:12-55 (ctypes.CDLL + explicit argtypes/restype, an int
status per call and an error string). Here the library holds no device, queue or buffers of its own: every call gets
raw device pointers of PyTorch tensors and the current HIP stream, and launches on it.
"""
import ctypes
from ctypes import c_char_p, c_float, c_int, c_longlong, c_size_t, c_void_p
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "librk_path.so"
HEADER = HERE.parent.parent / "include" / "rk_path.h"
ABI_VERSION = 17

RK_F32, RK_BF16 = 0, 1
RK_W_BF16, RK_W_INT8, RK_W_INT4 = 1, 2, 3
RK_X_PLAIN, RK_X_SILU_MUL, RK_X_RMS_NORM = 0, 1, 2
ERROR_NAMES = {1: "invalid argument", 2: "unsupported", 3: "workspace too small", 4: "HIP runtime error"}

P = c_void_p
# name -> (restype, argtypes); one entry per function declared in include/rk_path.h
SIGNATURES = {
    "rk_last_error": (c_char_p, []),
    "rk_clear_error": (None, []),
    "rk_abi_version": (c_int, []),
    "rk_device_info": (c_int, [P, c_char_p, c_int]),
    "rk_paged_decode_workspace_bytes": (c_size_t, [c_int] * 6),
    "rk_paged_decode": (c_int, [P, P, P, P, c_int, P, P] + [c_int] * 8 + [P, c_longlong, P, c_size_t, P]),
    "rk_paged_decode_phase": (c_int, [c_int, P, P, P, P, c_int, P, P] + [c_int] * 8
                              + [P, c_longlong, P, c_size_t, P, c_size_t, P]),
    "rk_paged_decode_plan_ints": (c_size_t, [c_int] * 6),
    "rk_paged_decode_plan": (c_int, [P, c_size_t, P, P] + [c_int] * 8 + [P]),
    "rk_paged_decode_planned": (c_int, [P, P, P, P, c_int, P, P] + [c_int] * 8
                                + [P, c_longlong, P, c_size_t, P, c_size_t, P]),
    "rk_paged_decode_noalloc_max_bytes": (c_size_t, []),
    "rk_paged_decode_noalloc": (c_int, [P, P, P, P, c_int, P, P] + [c_int] * 8 + [P, c_longlong, P]),
    "rk_kv_write": (c_int, [P, P, c_int, P, P, P, c_int] + [c_int] * 5 + [P]),
    "rk_kv_gather": (c_int, [P, P, P, P, c_int, P] + [c_int] * 7 + [P]),
    "rk_pages_init": (c_int, [P, P, P, P, c_int, c_int, c_int, P]),
    "rk_pages_advance": (c_int, [P, P, P, P] + [c_int] * 4 + [P, c_int, c_int, P, P, P]),
    "rk_pages_release": (c_int, [P, P, P, P] + [c_int] * 4 + [P, c_int, P]),
    "rk_pages_gather": (c_int, [P, P, c_int, c_int, c_int, P, c_int, c_int, P, P]),
    "rk_deltanet_decode": (c_int, [P] * 5 + [c_longlong] * 3 + [P] * 7 + [c_int] * 7 + [c_float, P]),
    "rk_paged_prefill": (c_int, [P, P, c_int, P, P, c_int, P, P, c_int, P, c_int, P, P, P] + [c_int] * 8
                         + [P, c_int, c_int, c_int, c_int, c_int, P, c_size_t, P, c_size_t, P]),
    "rk_paged_prefill_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "rk_paged_prefill_counters": (c_size_t, [c_int, c_int]),
    "rk_gated_delta_workspace_bytes": (c_size_t, [c_int, c_int]),
    "rk_gated_delta_chunked": (c_int, [P, P, c_longlong, P, P, P, c_int, P, P, P, P, P] + [c_int] * 5
                               + [P, c_size_t, P]),
    "rk_causal_conv1d": (c_int, [P, P, P, c_int, c_longlong, P, P, c_int, c_int, c_int, P]),
    "rk_deltanet_prefill_front": (c_int, [P] * 8 + [c_int, c_longlong, P, c_longlong] + [P] * 5 + [c_int] * 6
                                  + [P]),
    "rk_rms_norm_gated": (c_int, [P, P, P, c_int, c_longlong, c_int, P, c_int, c_int, c_float, P]),
    "rk_attn_prep": (c_int, [P, P, P, P, P, c_int, P, c_int, c_int, P, c_int, c_longlong, P, P, c_float, P, P]
                     + [c_int] * 5 + [P]),
    "rk_linear_workspace_bytes": (c_size_t, [c_int] * 4),
    "rk_linear_rows": (c_int, [P, P, c_int, c_int, c_int, P, c_int, P, P, P, P, P, c_size_t, P, c_int, P]),
    "rk_dequant_rows": (c_int, [P, P, c_int, P, P, P, c_int, c_int, c_int, c_int, P]),
    "rk_linear_rows_ex": (c_int, [P, P, c_longlong, c_int, P, c_longlong, c_int, c_int, c_int, P, c_int, P, P, P, P, P,
                                  c_size_t, P, c_int, P]),
    "rk_linear_rows_ex2": (c_int, [P, P, P, c_longlong, c_int, P, c_longlong, P, c_float, c_int, c_int, c_int, P, c_int,
                                   P, P, P, P, P, c_size_t, P, c_int, P]),
    "rk_swiglu_rows": (c_int, [P, P, c_longlong, c_int, P, c_longlong, P, c_float, c_int, c_int, c_int, P, c_int, P, P,
                               P, c_size_t, P, c_int, P]),
    "rk_rms_norm": (c_int, [P, P, c_int, c_longlong, P, c_int, c_int, c_int, c_float, P]),
    "rk_layer_norm": (c_int, [P, P, c_int, c_longlong, P, c_int, c_int, c_int, c_float, P]),
    "rk_rope": (c_int, [P, P, P, P, c_int, c_int, c_int, P]),
    "rk_silu_mul": (c_int, [P, P, c_longlong, P, c_longlong, c_int, c_int, P]),
}


PROBE_LIB_PATH = HERE / "librk_probe.so"
# the measurement probes of include/rk_probe.h (their library also exports rk_last_error)
PROBE_SIGNATURES = {
    "rk_probe_block_stream": (c_int, [P, P, P, c_int, c_int, c_int, c_int, P, P]),
    "rk_probe_state_rmw": (c_int, [P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_float, P]),
}


class RocmKernelError(RuntimeError):
    """A C-ABI call returned a nonzero status."""


class NativeRocm:
    """The loaded library with typed entry points. call(name, *args) raises RocmKernelError on a nonzero status."""

    def __init__(self, path: Path = LIB_PATH, signatures: dict = SIGNATURES):
        if not Path(path).exists():
            raise FileNotFoundError(f"{path} is missing: build it with `python metal-inference-engine_amd/native/build.py` "
                                    "(or __graft_entry__.build())")
        lib = ctypes.CDLL(str(path))
        for name, (res, args) in {**signatures, "rk_last_error": SIGNATURES["rk_last_error"],
                                  "rk_abi_version": SIGNATURES["rk_abi_version"]}.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.rk_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{path}: ABI version {lib.rk_abi_version()}, expected {ABI_VERSION}")
        self.lib = lib
        self.path = Path(path)

    def call(self, name: str, *args) -> None:
        rc = getattr(self.lib, name)(*args)
        if rc != 0:
            msg = self.lib.rk_last_error().decode(errors="replace")
            raise RocmKernelError(f"{name}: {ERROR_NAMES.get(rc, rc)}: {msg}")

    def last_error(self) -> str:
        return self.lib.rk_last_error().decode(errors="replace")


_lib: NativeRocm | None = None


def load() -> NativeRocm:
    """The process-wide library instance (loaded on first use; raises if the .so is missing)."""
    global _lib
    if _lib is None:
        _lib = NativeRocm()
    return _lib


_probes: NativeRocm | None = None


def load_probes() -> NativeRocm:
    """The measurement-probe library (librk_probe.so), loaded on first use."""
    global _probes
    if _probes is None:
        _probes = NativeRocm(PROBE_LIB_PATH, PROBE_SIGNATURES)
    return _probes
