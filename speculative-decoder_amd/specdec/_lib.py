"""ctypes binding of libspecdec.so.  Every symbol of include/specdec.h is
declared here with its argument types; `lib()` loads the library once."""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_int32, c_int64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libspecdec.so")

P = c_void_p
I32 = c_int32
I64 = c_int64

# name -> argument types (all return int)
SIGNATURES: dict[str, list] = {
    "specdec_abi_version": [],
    "specdec_probabilities": [P, c_int, I64, I64, I64, c_float, P, I64, P, I64, P],
    "specdec_accept_workspace": [I64, P],
    "specdec_accept_reject": [P, P, c_int, I64, I64, I64, I64, P, P, P, I64, I64, I64, P, P, I64, I32, P],
    "specdec_accept_reject_logits": [P, P, c_int, I64, I64, I64, I64, c_float, P, P, P, I64, I64, I64, P, P, I64,
                                     I32, P],
    "specdec_accept_count": [P, P, c_int, I64, I64, I64, I64, P, P, I64, I64, I64, P, P],
    "specdec_sample_inverse_cdf": [P, c_int, I64, I64, I64, P, P, P],
    "specdec_one_hot": [P, I64, I64, P, P],
    "specdec_ngram_lookup": [P, I64, P, I64, I32, I32, P, P, P],
    "specdec_block_plan": [P, I64, P, P, I64, I32, P, I32, I32, P, P],
    "specdec_block_free_checked": [P, P, I64, I32, I32, P, P],
    "specdec_block_slots": [P, I64, I64, I32, P, P],
    "specdec_slot_map": [P, I64, P, I32, I32, I32, I32, P, P, P, P, P],
    "specdec_rope_append": [P, c_int, I64, I32, I32, I32, P, P, I64, P, I32, I32, P, I64, I32, P, P, P],
    "specdec_kv_write": [P, P, c_int, I32, I32, P, I32, I32, P, I64, I32, P, P, P],
    "specdec_kv_gather": [P, P, c_int, I32, I32, P, I32, P, I64, I32, I32, P, P, P],
    "specdec_add_rmsnorm": [P, P, P, P, c_int, I64, I64, c_float, P],
    "specdec_silu_mul": [P, P, c_int, I64, I64, P],
    "specdec_rms_silu_mul": [P, P, P, c_int, I64, I64, I64, c_float, P],
    "specdec_attention_workspace": [I32, I32, I32, I32, I32, I32, I32, P],
    "specdec_attention_split": [I32, I32, I32, I32, I32],
    "specdec_paged_attention": [P, c_int, I64, P, P, P, I64, P, I32, I32, I32, I32, I32, I32, c_float,
                                I32, I32, P, I64, P, I64, P],
    "specdec_rope_paged_attention": [P, c_int, I64, P, P, P, I64, c_float, P, P, P, I64, P, I32, I32, I32, I32, I32,
                                     I32, c_float, I32, I32, P, I64, P, I64, P],
    "specdec_rope_paged_attention_parts": [P, I64, P, P, P, I64, c_float, P, P, P, I64, P, I32, I32, I32, I32, I32,
                                           c_float, I32, I32, P, P],
    "specdec_linear_attn_parts": [P, I64, I64, I32, P, I64, I32, I64, P, I64, I32, P, P],
    "specdec_head_workspace": [P],
    "specdec_head_logits": [P, I64, P, I64, I64, I64, I64, P, I64, P],
    "specdec_linear": [P, I64, P, I64, I32, I64, I64, I64, P, I64, I32, P],
    "specdec_linear_silu": [P, I64, P, I64, I32, I64, I64, I64, P, I64, I64, c_float, P, I64, P],
    "specdec_head_probabilities": [P, I64, P, I64, I64, I64, I64, c_float, P, I64, P, I64, P, I64, P, I64, I32, P],
    "specdec_paged_attention_static": [P, c_int, I64, P, P, P, I64, P, I32, I32, I32, I32, I32, I32, c_float,
                                       I32, I32, P, I64, P],
}

# fp32 split partials the library holds per GPU for specdec_paged_attention_static
STATIC_PARTIAL_FLOATS = 2 * 1024 * 1024

ABI_VERSION = 15
_lib: ctypes.CDLL | None = None


def available() -> bool:
    return LIB_PATH.exists()


HIP_DEVICE_SCHEDULE_SPIN = 1  # hipDeviceScheduleSpin


def spin_wait() -> bool:
    """Have HIP spin, not sleep, while the host waits for the GPU (a
    synchronising copy, an event or a stream wait), so the host resumes as
    soon as the GPU is done -- a round loop reads each verdict back this
    way -- at the cost of a busy core while it waits.  It must run before the
    process first uses the GPU (torch.cuda.is_available() already does);
    returns whether HIP accepted it.  Off unless called."""
    for name in ("libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
        try:
            hip = ctypes.CDLL(name)
            break
        except OSError:
            continue
    else:
        return False
    hip.hipSetDeviceFlags.argtypes = [ctypes.c_uint]
    hip.hipSetDeviceFlags.restype = c_int
    return hip.hipSetDeviceFlags(HIP_DEVICE_SCHEDULE_SPIN) == 0


def load(path: Path = LIB_PATH) -> ctypes.CDLL:
    """Load the library and declare every entry point (no GPU needed)."""
    handle = ctypes.CDLL(str(path))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes = argtypes
        fn.restype = c_int
    version = handle.specdec_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}; rebuild it")
    return handle


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built: the hot path has no CPU fallback. "
                "Build it with `python speculative-decoder_amd/specdec/build.py`."
            )
        _lib = load()
    return _lib
