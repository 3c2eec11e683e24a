"""ctypes binding of libtrk.so, the C ABI declared in include/trk.h.

The library is loaded once per process from the package directory. It is never built or
replaced at load time: a missing or mismatched library raises, so a GPU run cannot silently
take another path.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIBRARY = Path(__file__).resolve().parent / "libtrk.so"
ABI_VERSION = 4

DTYPE_F16, DTYPE_BF16, DTYPE_F32 = 0, 1, 2
KERNEL_GENERIC, KERNEL_MFMA = 0, 1
EPI_STORE, EPI_F32, EPI_ADD, EPI_SILU_MUL = 0, 1, 2, 3

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP, ERR_NOMEM = 0, 1, 2, 3, 4

# Every symbol include/trk.h declares, with (restype, argtypes).
_c_int, _c_void_p, _c_size_t, _c_char_p = ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_char_p
_int3 = ctypes.c_int * 3


class VariantInfo(ctypes.Structure):
    """struct trk_variant_info."""

    _fields_ = [
        ("name", ctypes.c_char * 64),
        ("kind", ctypes.c_int),
        ("order", ctypes.c_int * 3),
        ("tile", ctypes.c_int * 5),
        ("grid", ctypes.c_int * 3),
        ("block", ctypes.c_int),
        ("lds_bytes", ctypes.c_int),
        ("t_min", ctypes.c_int),
        ("t_max", ctypes.c_int),
        ("flops", ctypes.c_double),
        ("bytes", ctypes.c_double),
        ("packed_offset", ctypes.c_size_t * 3),
    ]

    def as_dict(self) -> dict:
        return {
            "name": self.name.decode(), "kind": "mfma" if self.kind == KERNEL_MFMA else "generic",
            "order": list(self.order), "tile": list(self.tile), "grid": list(self.grid),
            "block": self.block, "lds_bytes": self.lds_bytes, "t_min": self.t_min,
            "t_max": self.t_max, "flops": self.flops, "bytes": self.bytes,
            "packed_offset": list(self.packed_offset),
        }


SIGNATURES = {
    "trk_abi_version": (_c_int, []),
    "trk_last_error": (_c_char_p, []),
    "trk_plan_create": (_c_int, [_int3, _int3, _c_int, _c_int, ctypes.POINTER(_c_void_p)]),
    "trk_plan_create_padded": (_c_int, [_int3, _int3, _c_int, _c_int, _c_int,
                                        ctypes.POINTER(_c_void_p)]),
    "trk_plan_load_module": (_c_int, [_c_void_p, _c_char_p, ctypes.POINTER(_c_int)]),
    "trk_plan_destroy": (None, [_c_void_p]),
    "trk_plan_packed_bytes": (_c_size_t, [_c_void_p]),
    "trk_plan_variant_count": (_c_int, [_c_void_p]),
    "trk_plan_select": (_c_int, [_c_void_p, _c_int]),
    "trk_plan_describe": (_c_int, [_c_void_p, _c_int, _c_int, ctypes.POINTER(VariantInfo)]),
    "trk_plan_set_variant": (_c_int, [_c_void_p, _c_int, _c_int, _c_int]),
    "trk_pack": (_c_int, [_c_void_p] * 6),
    "trk_forward": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_void_p]),
    "trk_forward_variant": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_int,
                                     _c_void_p]),
    "trk_forward_epilogue": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_int,
                                      _c_int, _c_void_p, _c_int, _c_void_p]),
    "trk_forward_swiglu": (_c_int, [_c_void_p] * 6 + [_c_int, _c_void_p]),
    "trk_consume_silu_mul": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int, _c_size_t,
                                      _c_void_p]),
    "trk_consume_add": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int, _c_size_t, _c_void_p]),
    "trk_empty_launch": (_c_int, [_c_void_p]),
    "trk_empty_launch_args": (_c_int, [_c_void_p]),
    "trk_empty_call": (_c_int, []),
}

_lib = None


class TrkError(RuntimeError):
    """A libtrk call returned a non-zero status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"libtrk status {status}: {message}")
        self.status = status


def load() -> ctypes.CDLL:
    """Load libtrk.so (once) and bind every declared symbol; raise if it is missing."""
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            raise RuntimeError(
                f"{LIBRARY} is not built; run `python -m factorized_inference.build_ext` "
                "(or __graft_entry__.build()) first")
        lib = ctypes.CDLL(str(LIBRARY))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.trk_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libtrk ABI {version}, expected {ABI_VERSION}")
        _lib = lib
    return _lib


def check(status: int) -> None:
    if status != OK:
        raise TrkError(status, load().trk_last_error().decode())


class Plan:
    """Owner of one trk_plan (host memory only). kernel_rank > rank makes a padded plan
    (trk_plan_create_padded): its kernels run at kernel_rank on zero-padded cores."""

    def __init__(self, input_modes, output_modes, rank: int, dtype_code: int,
                 kernel_rank: int | None = None):
        lib = load()
        handle = _c_void_p()
        self.rank = int(rank)
        self.kernel_rank = int(kernel_rank or rank)
        check(lib.trk_plan_create_padded(_int3(*input_modes), _int3(*output_modes), self.rank,
                                         self.kernel_rank, int(dtype_code), ctypes.byref(handle)))
        self._lib = lib
        self.handle = handle.value
        self.modules: list[str] = []

    def __del__(self):
        handle, self.handle = getattr(self, "handle", None), None
        if handle:
            self._lib.trk_plan_destroy(handle)

    @property
    def packed_bytes(self) -> int:
        return int(self._lib.trk_plan_packed_bytes(self.handle))

    @property
    def variant_count(self) -> int:
        return int(self._lib.trk_plan_variant_count(self.handle))

    def select(self, tokens: int) -> int:
        return int(self._lib.trk_plan_select(self.handle, int(tokens)))

    def describe(self, variant: int = -1, tokens: int = 1) -> dict:
        info = VariantInfo()
        check(self._lib.trk_plan_describe(self.handle, int(variant), int(tokens),
                                          ctypes.byref(info)))
        return info.as_dict()

    def variants(self, tokens: int = 1) -> list[dict]:
        return [self.describe(v, tokens) for v in range(self.variant_count)]

    def set_variant(self, t_min: int, t_max: int, variant: int) -> None:
        check(self._lib.trk_plan_set_variant(self.handle, int(t_min), int(t_max), int(variant)))

    @property
    def has_mfma(self) -> bool:
        return any(v["kind"] == "mfma" for v in self.variants())

    def load_module(self, path) -> int:
        """Add the variants of a variant module (trk_plan_load_module); returns how many.
        Call before packing: the variants may add packed sections."""
        added = _c_int(0)
        check(self._lib.trk_plan_load_module(self.handle, str(path).encode(), ctypes.byref(added)))
        self.modules.append(str(path))
        return added.value
