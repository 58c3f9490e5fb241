"""ctypes binding of libnimbus_attn.so (declared in include/nimbus_attn.h).

The library is loaded after `import torch` so that its DT_NEEDED
libamdhip64.so.7 resolves to the HIP runtime torch already mapped: one
runtime, so torch's streams (including a capturing stream inside
torch.cuda.graph) are valid handles for the kernels.

There is no CPU or PyTorch fallback: if the library is missing or fails to
load, every entry point raises.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be imported before the library is loaded)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnimbus_attn.so")

NIMBUS_FLOAT16 = 0
NIMBUS_BFLOAT16 = 1
NIMBUS_ERR_INVALID = -1
NIMBUS_ERR_UNSUPPORTED = -2
NIMBUS_ERR_ALIGNMENT = -3
NIMBUS_ERR_WORKSPACE = -4
NIMBUS_ERR_SCRATCH = -5
NOALLOC_SCRATCH_BYTES = 64 << 20  # NIMBUS_NOALLOC_SCRATCH_BYTES
ABI_VERSION = 15

# Entry points and their C signatures, in the order include/nimbus_attn.h declares them.
_c_int, _c_i32, _c_i64, _c_p, _c_f = ctypes.c_int, ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p, ctypes.c_float
SIGNATURES = {
    "nimbus_attn_abi_version": (_c_int, []),
    "nimbus_attn_error_string": (ctypes.c_char_p, [_c_int]),
    "nimbus_write_kv": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i64, _c_i64, _c_i64,
                                 _c_i64, _c_i64, _c_i32, _c_p]),
    "nimbus_paged_decode_workspace_bytes": (_c_i64, [_c_i32, _c_i32, _c_i32, _c_i64]),
    "nimbus_paged_decode": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64,
                                     _c_i32, _c_p, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32,
                                     _c_i32, _c_i64, _c_f, _c_i32, _c_p]),
    "nimbus_paged_decode_pages": None,
    "nimbus_paged_decode_merge": None,
    "nimbus_paged_decode_noalloc": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p,
                                             _c_i64, _c_i32, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32,
                                             _c_i32, _c_i32, _c_i64, _c_f, _c_i32, _c_p]),
    "nimbus_paged_prefill": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64,
                                      _c_i32, _c_p, _c_p, _c_p, _c_p, _c_i32, _c_p, _c_i64, _c_i64, _c_i32, _c_i32,
                                      _c_i32, _c_i32, _c_f, _c_i32, _c_p]),
    "nimbus_paged_prefill_pieces_workspace_bytes": (_c_i64, [_c_i32, _c_i32, _c_i32]),
    "nimbus_paged_prefill_pieces": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p,
                                             _c_i64, _c_i32, _c_p, _c_p, _c_p, _c_i32, _c_p, _c_i32, _c_i32, _c_p,
                                             _c_i64, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_f,
                                             _c_i32, _c_p]),
    "nimbus_paged_prefill_stream_flag_bytes": (_c_i64, [_c_i32, _c_i32, _c_i32]),
    "nimbus_paged_prefill_stream_workspace_bytes": (_c_i64, [_c_i32, _c_i32, _c_i32, _c_i32]),
    "nimbus_paged_prefill_stream": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p,
                                             _c_i64, _c_i32, _c_p, _c_p, _c_p, _c_p, _c_i32, _c_p, _c_i64, _c_p,
                                             _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_f, _c_i32, _c_p]),
    "nimbus_paged_verify_workspace_bytes": (_c_i64, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i64]),
    "nimbus_paged_verify": None,
    "nimbus_add_rms_norm": (_c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i32,
                                     _c_f, _c_i32, _c_p]),
    "nimbus_add_rms_norm_partials": (_c_int, [_c_p, _c_i32, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_i64,
                                              _c_i64, _c_i32, _c_f, _c_i32, _c_p]),
    "nimbus_int8_matmul_workspace_bytes": (_c_i64, [_c_i64, _c_i32, _c_i32]),
    "nimbus_int8_matmul": (_c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_p,
                                    _c_i64, _c_i32, _c_p]),
    "nimbus_int8_packed_weight_bytes": (_c_i64, [_c_i32, _c_i32]),
    "nimbus_int8_pack_weight": (_c_int, [_c_p, _c_i64, _c_i32, _c_i32, _c_p, _c_p]),
    "nimbus_int8_matmul_packed_workspace_bytes": (_c_i64, [_c_i64, _c_i32, _c_i32]),
    "nimbus_int8_matmul_packed": (_c_int, [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_p,
                                           _c_i64, _c_i32, _c_p]),
    "nimbus_int8_matmul_packed_plan_workspace_bytes": (_c_i64, [_c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                                                _c_i32]),
    "nimbus_int8_matmul_packed_plan": (_c_int, [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32,
                                                _c_i32, _c_i32, _c_i32, _c_i32, _c_p, _c_i64, _c_i32, _c_p]),
    "nimbus_int8_matmul_packed_silu": (_c_int, [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32,
                                                _c_i32, _c_i32, _c_i32, _c_i32, _c_p]),
    "nimbus_int8_matmul_packed_partials": (_c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32,
                                                    _c_i32, _c_i32, _c_p, _c_i64, _c_i32, _c_p]),
    "nimbus_rope": (_c_int, [_c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_p]),
    "nimbus_rope_write_kv": (_c_int, [_c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_p, _c_p, _c_i64, _c_i32,
                                      _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_p]),
    "nimbus_silu_mul": (_c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_p]),
    "nimbus_greedy_step": (_c_int, [_c_p, _c_i64, _c_i32, _c_i32, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i32,
                                    _c_i32, _c_p, _c_p, _c_p, _c_i32, _c_i64, _c_p]),
}

SIGNATURES["nimbus_paged_decode_pages"] = SIGNATURES["nimbus_paged_decode"]
SIGNATURES["nimbus_paged_decode_merge"] = SIGNATURES["nimbus_paged_decode"]
SIGNATURES["nimbus_paged_verify"] = (_c_int, [_c_i32] + SIGNATURES["nimbus_paged_decode"][1])

_lib = None


class NimbusLibraryError(RuntimeError):
    pass


def load():
    """Returns the loaded library, loading it on first use."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise NimbusLibraryError(
            f"{LIB_PATH} is not built; run `python -m nimbus_amd.build` (there is no fallback path)")
    lib = ctypes.CDLL(LIB_PATH, mode=getattr(os, "RTLD_LOCAL", 0))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.nimbus_attn_abi_version() != ABI_VERSION:
        raise NimbusLibraryError(f"ABI version {lib.nimbus_attn_abi_version()} != {ABI_VERSION}")
    _lib = lib
    return lib


def hip_runtimes() -> list[str]:
    """Distinct libamdhip64 files mapped into this process (should be one)."""
    paths = set()
    with open("/proc/self/maps") as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 6 and "libamdhip64" in parts[5]:
                paths.add(os.path.realpath(parts[5]))
    return sorted(paths)


def check(rc: int, what: str) -> None:
    """Maps a non-zero return code of an entry point to a Python exception."""
    if rc == 0:
        return
    msg = f"{what}: {load().nimbus_attn_error_string(rc).decode()} (code {rc})"
    if rc == NIMBUS_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    if rc < 0:
        raise ValueError(msg)
    raise RuntimeError(msg)


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return NIMBUS_FLOAT16
    if dtype == torch.bfloat16:
        return NIMBUS_BFLOAT16
    raise NotImplementedError(f"dtype {dtype} is not supported (fp16 or bf16)")


def stream_of(t: torch.Tensor) -> int:
    """The raw handle of the current stream on t's device (the capture stream
    inside torch.cuda.graph), read without building a Stream object."""
    return torch._C._cuda_getCurrentRawStream(t.get_device())


