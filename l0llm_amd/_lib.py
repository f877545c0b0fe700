"""ctypes binding of libl0hip.so. Prototypes are read from include/l0hip.h so the binding and
the C ABI cannot drift apart. Loading fails loudly when the library has not been built: there
is no CPU fallback for any operation."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
HEADER = ROOT / "include" / "l0hip.h"
LIB_PATH = PKG / "libl0hip.so"

OK = 0
ERR_INVALID_ARG = -1
ERR_UNSUPPORTED = -2
ERR_INVALID_OP = -3
ERR_INVALID_DATA = -4
ERR_OUT_OF_MEMORY = -5
ERR_DEVICE = -6

F32, F16, BF16, I8PC = 0, 1, 2, 3
PRECISION_AUTO, PRECISION_FLOAT32, PRECISION_FLOAT16, PRECISION_INT8, PRECISION_BFLOAT16 = range(5)


class L0hError(Exception):
    """Base of the errors raised for a non-zero status of the C ABI."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class InvalidArgumentError(L0hError, ValueError):
    """ArgumentException / ArgumentNullException / ArgumentOutOfRangeException."""


class UnsupportedError(L0hError, NotImplementedError):
    """NotSupportedException."""


class InvalidOperationError(L0hError, RuntimeError):
    """InvalidOperationException."""


class InvalidDataError(L0hError, ValueError):
    """InvalidDataException."""


class DeviceOutOfMemoryError(L0hError, MemoryError):
    """Device allocation failure."""


class DeviceError(L0hError, RuntimeError):
    """HIP runtime or device failure."""


_ERRORS = {
    ERR_INVALID_ARG: InvalidArgumentError,
    ERR_UNSUPPORTED: UnsupportedError,
    ERR_INVALID_OP: InvalidOperationError,
    ERR_INVALID_DATA: InvalidDataError,
    ERR_OUT_OF_MEMORY: DeviceOutOfMemoryError,
    ERR_DEVICE: DeviceError,
}


class ModelConfig(ctypes.Structure):
    """l0h_model_config (the HfModelConfig fields the path uses, HfModelConfig.cs:10-120)."""

    _fields_ = [
        ("hidden_size", ctypes.c_int),
        ("intermediate_size", ctypes.c_int),
        ("num_layers", ctypes.c_int),
        ("num_attention_heads", ctypes.c_int),
        ("num_key_value_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("vocab_size", ctypes.c_int),
        ("max_position_embeddings", ctypes.c_int),
        ("rms_norm_eps", ctypes.c_float),
        ("rope_theta", ctypes.c_double),
        ("attention_bias", ctypes.c_int),
        ("tie_word_embeddings", ctypes.c_int),
        ("rope_type", ctypes.c_int),
        ("rope_factor", ctypes.c_double),
        ("rope_original_max_position_embeddings", ctypes.c_int),
        ("rope_beta_fast", ctypes.c_double),
        ("rope_beta_slow", ctypes.c_double),
        ("rope_mscale", ctypes.c_double),
        ("rope_mscale_all_dim", ctypes.c_double),
        ("rope_attention_factor", ctypes.c_double),
        ("rope_low_freq_factor", ctypes.c_double),
        ("rope_high_freq_factor", ctypes.c_double),
        ("rope_truncate", ctypes.c_int),
    ]


_SCALARS = {
    "int": ctypes.c_int,
    "float": ctypes.c_float,
    "double": ctypes.c_double,
    "size_t": ctypes.c_size_t,
    "uint64_t": ctypes.c_uint64,
    "l0h_probe_fn": ctypes.c_void_p,
    "void": None,
}

# void (*)(void* user, int layer, const char* stage, const float* values, int count)
PROBE_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float),
                            ctypes.c_int)

_DECL = re.compile(r"^(int|const char\*)\s+(l0h_\w+)\(([^;]*)\);", re.M | re.S)


def declared_functions(header: Path = HEADER) -> dict[str, tuple[str, list[str]]]:
    """Function name -> (return type, parameter declarations) for every l0h_ entry point."""
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    out: dict[str, tuple[str, list[str]]] = {}
    for ret, name, params in _DECL.findall(text):
        plist = [p.strip() for p in " ".join(params.split()).split(",") if p.strip()]
        if plist == ["void"]:
            plist = []
        out[name] = (ret, plist)
    return out


def _ctype(param: str):
    if "*" in param:
        return ctypes.c_void_p
    base = param.replace("const ", "").split()[0]
    if base not in _SCALARS:
        raise TypeError(f"unmapped parameter type in l0hip.h: {param}")
    return _SCALARS[base]


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python l0llm_amd/build.py` (hipcc, gfx950). "
            "There is no CPU fallback.")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (ret, params) in declared_functions().items():
        fn = getattr(lib, name)
        fn.restype = ctypes.c_char_p if ret == "const char*" else ctypes.c_int
        fn.argtypes = [_ctype(p) for p in params]
    return lib


lib = _load()


def check(status: int) -> None:
    """Raises the exception matching a non-zero status, with the library's message."""
    if status != OK:
        msg = lib.l0h_last_error().decode(errors="replace")
        raise _ERRORS.get(status, L0hError)(status, msg or f"status {status}")
