"""ctypes binding of libsfa.so (the C ABI declared in include/sfa.h).

The library is loaded from the package directory (built in-tree by
``python -m ops_amd.build``).  Loading fails loudly: there is no fallback of
any kind when the library or a GPU is missing.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libsfa.so"

SFA_ABI_VERSION = 2
SFA_DTYPE_F32 = 0
SFA_DTYPE_BF16 = 1
SFA_DTYPE_FP8_E4M3 = 2
SFA_DKV_AUTO = 0
SFA_DKV_ATOMIC = 1
SFA_DKV_CSR = 2
SFA_BWD_MERGE_KV = 1  # sfa_bwd_args.flags: dk receives dK + dV of rows k and v share
SFA_FWD_IDX_SORTED = 1  # sfa_fwd_args.flags: index rows are ascending (no sort pass before the MLA prefill)

SFA_OK = 0
SFA_E_INVALID = -1
SFA_E_WORKSPACE = -2
SFA_E_UNSUPPORTED = -3
SFA_E_HIP = -4

SFA_NOALLOC_SCRATCH_BYTES = 64 << 20

EXPORTED_SYMBOLS = (
    "sfa_abi_version",
    "sfa_last_error",
    "sfa_fwd_workspace_size",
    "sfa_fwd",
    "sfa_fwd_noalloc",
    "sfa_bwd_workspace_size",
    "sfa_bwd",
    "sfa_fwd_paged_workspace_size",
    "sfa_fwd_paged",
    "sfa_indexer_topk_workspace_size",
    "sfa_indexer_topk",
)

_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


class FwdArgs(ctypes.Structure):
    """Mirror of ``sfa_fwd_args``."""
    _fields_ = [
        ("dtype", _i32),
        ("B", _i32), ("Sq", _i32), ("Skv", _i32), ("Hq", _i32), ("Hkv", _i32),
        ("Dqk", _i32), ("Dv", _i32), ("topk", _i32),
        ("scale", ctypes.c_float),
        ("q", _vp), ("q_sb", _i64), ("q_ss", _i64), ("q_sh", _i64),
        ("k", _vp), ("k_sb", _i64), ("k_ss", _i64), ("k_sh", _i64),
        ("v", _vp), ("v_sb", _i64), ("v_ss", _i64), ("v_sh", _i64),
        ("idx", _vp), ("i_sb", _i64), ("i_ss", _i64), ("i_sh", _i64),
        ("kv_lens", _vp),
        ("sink", _vp),
        ("out", _vp), ("o_sb", _i64), ("o_ss", _i64), ("o_sh", _i64),
        ("lse", _vp), ("l_sb", _i64), ("l_ss", _i64), ("l_sh", _i64),
        ("num_splits", _i32),
        ("flags", _i32),
    ]


class BwdArgs(ctypes.Structure):
    """Mirror of ``sfa_bwd_args``."""
    _fields_ = [
        ("fwd", FwdArgs),
        ("dout", _vp), ("do_sb", _i64), ("do_ss", _i64), ("do_sh", _i64),
        ("dq", _vp), ("dq_sb", _i64), ("dq_ss", _i64), ("dq_sh", _i64),
        ("dk", _vp), ("dk_sb", _i64), ("dk_ss", _i64), ("dk_sh", _i64),
        ("dv", _vp), ("dv_sb", _i64), ("dv_ss", _i64), ("dv_sh", _i64),
        ("dlse", _vp),
        ("dsink", _vp),
        ("dkv_mode", _i32),
        ("flags", _i32),
    ]


class KvPages(ctypes.Structure):
    """Mirror of ``sfa_kv_pages``."""
    _fields_ = [
        ("block_table", _vp), ("bt_sb", _i64),
        ("max_pages", _i32), ("page_size", _i32), ("num_pages", _i32), ("flags", _i32),
    ]


class IndexerArgs(ctypes.Structure):
    """Mirror of ``sfa_indexer_args``."""
    _fields_ = [
        ("B", _i32), ("Sq", _i32), ("Skv", _i32), ("H", _i32), ("D", _i32), ("topk", _i32),
        ("dtype", _i32),
        ("q", _vp), ("q_sb", _i64), ("q_ss", _i64), ("q_sh", _i64),
        ("k", _vp), ("k_sb", _i64), ("k_ss", _i64),
        ("k_scale", _vp), ("ks_sb", _i64),
        ("w", _vp), ("w_sb", _i64), ("w_ss", _i64),
        ("kv_lens", _vp),
        ("idx", _vp), ("i_sb", _i64), ("i_ss", _i64),
        ("logits", _vp), ("g_sb", _i64), ("g_ss", _i64),
        ("flags", _i32),
    ]


class SFAError(RuntimeError):
    """A failure reported by libsfa (HIP runtime or unsupported request)."""


_lock = threading.Lock()
_lib = None


def lib_path() -> Path:
    return Path(os.environ.get("SFA_LIB", str(LIB_PATH)))


def load() -> ctypes.CDLL:
    """Load libsfa.so once; raises if it is missing or has the wrong ABI."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = lib_path()
        if not path.exists():
            raise SFAError(f"{path} is missing: build it with `python -m ops_amd.build`")
        lib = ctypes.CDLL(str(path))
        lib.sfa_abi_version.restype = ctypes.c_int
        lib.sfa_abi_version.argtypes = []
        lib.sfa_last_error.restype = ctypes.c_char_p
        lib.sfa_last_error.argtypes = []
        lib.sfa_fwd_workspace_size.restype = ctypes.c_size_t
        lib.sfa_fwd_workspace_size.argtypes = [ctypes.POINTER(FwdArgs)]
        lib.sfa_fwd.restype = ctypes.c_int
        lib.sfa_fwd.argtypes = [ctypes.POINTER(FwdArgs), _vp, ctypes.c_size_t, _vp]
        lib.sfa_fwd_noalloc.restype = ctypes.c_int
        lib.sfa_fwd_noalloc.argtypes = [ctypes.POINTER(FwdArgs), _vp]
        lib.sfa_bwd_workspace_size.restype = ctypes.c_size_t
        lib.sfa_bwd_workspace_size.argtypes = [ctypes.POINTER(BwdArgs)]
        lib.sfa_bwd.restype = ctypes.c_int
        lib.sfa_bwd.argtypes = [ctypes.POINTER(BwdArgs), _vp, ctypes.c_size_t, _vp]
        lib.sfa_fwd_paged_workspace_size.restype = ctypes.c_size_t
        lib.sfa_fwd_paged_workspace_size.argtypes = [ctypes.POINTER(FwdArgs), ctypes.POINTER(KvPages)]
        lib.sfa_fwd_paged.restype = ctypes.c_int
        lib.sfa_fwd_paged.argtypes = [ctypes.POINTER(FwdArgs), ctypes.POINTER(KvPages), _vp, ctypes.c_size_t, _vp]
        lib.sfa_indexer_topk_workspace_size.restype = ctypes.c_size_t
        lib.sfa_indexer_topk_workspace_size.argtypes = [ctypes.POINTER(IndexerArgs)]
        lib.sfa_indexer_topk.restype = ctypes.c_int
        lib.sfa_indexer_topk.argtypes = [ctypes.POINTER(IndexerArgs), _vp, ctypes.c_size_t, _vp]
        ver = lib.sfa_abi_version()
        if ver != SFA_ABI_VERSION:
            raise SFAError(f"libsfa ABI version {ver} != expected {SFA_ABI_VERSION}; rebuild")
        _lib = lib
        return lib


def check(rc: int) -> None:
    """Map a libsfa return code to a Python exception."""
    if rc == SFA_OK:
        return
    msg = (_lib.sfa_last_error() or b"").decode(errors="replace") if _lib is not None else ""
    if rc == SFA_E_INVALID:
        raise ValueError(msg)
    raise SFAError(f"libsfa error {rc}: {msg}")
