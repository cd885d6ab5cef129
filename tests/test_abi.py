"""C ABI checks that need no GPU: the library loads, exports every symbol
include/sfa.h declares, its argument structs match the header byte for byte,
and invalid arguments come back as error codes (no HIP call is made before
validation)."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from ops_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "sfa.h"


def _declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"SFA_API\s+[\w\s\*]+?\b(sfa_\w+)\s*\(", text)))


def test_header_declares_expected_symbols():
    assert _declared_functions() == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.lib_path())], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    for name in _declared_functions():
        assert name in exported, name
        assert hasattr(lib, name)
    assert lib.sfa_abi_version() == _lib.SFA_ABI_VERSION


def test_struct_layout_matches_header(tmp_path):
    src = tmp_path / "layout.c"
    fields_f = [f for f, _ in _lib.FwdArgs._fields_]
    fields_b = [f for f, _ in _lib.BwdArgs._fields_]
    fields_p = [f for f, _ in _lib.KvPages._fields_]
    fields_i = [f for f, _ in _lib.IndexerArgs._fields_]
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {",
             'printf("%zu %zu %zu %zu\\n", sizeof(sfa_fwd_args), sizeof(sfa_bwd_args), sizeof(sfa_kv_pages), '
             'sizeof(sfa_indexer_args));']
    lines += [f'printf("%zu\\n", offsetof(sfa_fwd_args, {f}));' for f in fields_f]
    lines += [f'printf("%zu\\n", offsetof(sfa_bwd_args, {f}));' for f in fields_b]
    lines += [f'printf("%zu\\n", offsetof(sfa_kv_pages, {f}));' for f in fields_p]
    lines += [f'printf("%zu\\n", offsetof(sfa_indexer_args, {f}));' for f in fields_i]
    lines += ["return 0; }"]
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-o", str(exe), str(src)], check=True)
    vals = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    assert int(vals[0]) == ctypes.sizeof(_lib.FwdArgs)
    assert int(vals[1]) == ctypes.sizeof(_lib.BwdArgs)
    assert int(vals[2]) == ctypes.sizeof(_lib.KvPages)
    assert int(vals[3]) == ctypes.sizeof(_lib.IndexerArgs)
    offs = [int(x) for x in vals[4:]]
    py = ([getattr(_lib.FwdArgs, f).offset for f in fields_f] + [getattr(_lib.BwdArgs, f).offset for f in fields_b]
          + [getattr(_lib.KvPages, f).offset for f in fields_p] + [getattr(_lib.IndexerArgs, f).offset for f in fields_i])
    assert offs == py


def _valid_args():
    a = _lib.FwdArgs()
    a.dtype = _lib.SFA_DTYPE_BF16
    a.B, a.Sq, a.Skv, a.Hq, a.Hkv, a.Dqk, a.Dv, a.topk = 1, 4, 8, 16, 1, 128, 128, 32
    a.scale = 0.0
    for name in ("q", "k", "v", "idx", "out", "lse"):
        setattr(a, name, 0x10000)
    return a


@pytest.mark.parametrize("field,value", [
    ("topk", 0), ("topk", -3), ("Hkv", 3), ("B", 0), ("Dqk", 0), ("Dqk", 5000), ("dtype", 7), ("num_splits", -1),
    ("flags", 2), ("flags", -1), ("q", None),
])
def test_invalid_arguments_are_rejected(field, value):
    lib = _lib.load()
    a = _valid_args()
    setattr(a, field, value)
    rc = lib.sfa_fwd(ctypes.byref(a), None, 0, None)
    assert rc == _lib.SFA_E_INVALID
    assert lib.sfa_last_error()
    with pytest.raises(ValueError):
        _lib.check(rc)
    assert lib.sfa_fwd_workspace_size(ctypes.byref(a)) == 0


def test_null_struct_is_rejected():
    lib = _lib.load()
    assert lib.sfa_fwd(None, None, 0, None) == _lib.SFA_E_INVALID
    assert lib.sfa_bwd(None, None, 0, None) == _lib.SFA_E_INVALID


def test_workspace_sizes_follow_the_plan():
    lib = _lib.load()
    a = _valid_args()
    assert lib.sfa_fwd_workspace_size(ctypes.byref(a)) == 0  # generic / not split
    # decode-shaped MLA: split-k partials (fp32 O + LSE per split)
    a.B, a.Sq, a.Skv, a.Hq, a.Hkv, a.Dqk, a.Dv, a.topk = 64, 1, 65536, 128, 1, 576, 512, 2048
    a.k_ss = a.v_ss = 576
    a.k_sh = a.v_sh = 576
    a.k_sb = a.v_sb = 65536 * 576
    a.q_sh, a.q_ss, a.q_sb = 576, 128 * 576, 128 * 576
    a.o_sh, a.o_ss, a.o_sb = 512, 128 * 512, 128 * 512
    a.v = a.k
    ws = lib.sfa_fwd_workspace_size(ctypes.byref(a))
    splits = ws // (64 * 128 * 512 * 4)
    assert splits >= 2 and ws >= splits * 64 * 128 * (512 + 1) * 4
    b = _lib.BwdArgs()
    b.fwd = _valid_args()
    need = lib.sfa_bwd_workspace_size(ctypes.byref(b))
    assert need >= (8 * 128 * 2 + 4 * 16) * 4


def _mla_prefill_args(S, K, Skv=None):
    a = _valid_args()
    Skv = S if Skv is None else Skv
    a.B, a.Sq, a.Skv, a.Hq, a.Hkv, a.Dqk, a.Dv, a.topk = 1, S, Skv, 128, 1, 576, 512, K
    a.k_ss = a.v_ss = a.k_sh = a.v_sh = 576
    a.k_sb = a.v_sb = Skv * 576
    a.q_sh, a.q_ss, a.q_sb = 576, 128 * 576, S * 128 * 576
    a.o_sh, a.o_ss, a.o_sb = 512, 128 * 512, S * 128 * 512
    a.v = a.k
    a.i_sh, a.i_ss, a.i_sb = K, K, S * K
    return a


def test_persistent_prefill_workspace_holds_sorted_index_rows():
    """The persistent MLA prefill (>= 4096 work items) takes 256 bytes of
    claim counters plus its index rows in ascending order (B*Sq*Hkv*topk
    int32) unless SFA_FWD_IDX_SORTED declares them sorted; fewer items (the
    plain grid) or Skv beyond the sort's 65536-key bitmap take no sorted
    copy."""
    lib = _lib.load()
    a = _mla_prefill_args(32768, 2048)
    rows = 32768 * 2048 * 4
    assert lib.sfa_fwd_workspace_size(ctypes.byref(a)) == 256 + rows
    a.flags = _lib.SFA_FWD_IDX_SORTED
    assert lib.sfa_fwd_workspace_size(ctypes.byref(a)) == 256
    a = _mla_prefill_args(4096, 100)  # rows padded to 256 bytes
    assert lib.sfa_fwd_workspace_size(ctypes.byref(a)) == 256 + (4096 * 100 * 4 + 255) // 256 * 256
    a = _mla_prefill_args(4000, 2048)  # plain grid: no counters, no sort
    assert lib.sfa_fwd_workspace_size(ctypes.byref(a)) == 0
    a = _mla_prefill_args(4096, 2048, Skv=70000)
    assert lib.sfa_fwd_workspace_size(ctypes.byref(a)) == 256
    a = _mla_prefill_args(4096, 4096)  # top-k beyond the sort's 2048 slots (two splits of 2048)
    assert lib.sfa_fwd_workspace_size(ctypes.byref(a)) > 0
    # paged: the rows hold logical keys, sorted the same way
    a = _mla_prefill_args(8192, 2048)
    a.k_sb = a.v_sb = 64 * 576  # 64-row pages
    pg = _lib.KvPages()
    pg.block_table, pg.bt_sb, pg.max_pages, pg.page_size, pg.num_pages, pg.flags = 0x10000, 128, 128, 64, 128, 0
    assert lib.sfa_fwd_paged_workspace_size(ctypes.byref(a), ctypes.byref(pg)) == 256 + 8192 * 2048 * 4
    a.flags = _lib.SFA_FWD_IDX_SORTED
    assert lib.sfa_fwd_paged_workspace_size(ctypes.byref(a), ctypes.byref(pg)) == 256


def test_bwd_rejects_missing_gradients_and_csr_mode():
    lib = _lib.load()
    b = _lib.BwdArgs()
    b.fwd = _valid_args()
    assert lib.sfa_bwd(ctypes.byref(b), None, 0, None) == _lib.SFA_E_INVALID  # null dq/dk/dv
    for name in ("dout", "dq", "dk", "dv"):
        setattr(b, name, 0x10000)
    b.dkv_mode = 9
    assert lib.sfa_bwd(ctypes.byref(b), None, 0, None) == _lib.SFA_E_INVALID
    b.dkv_mode = _lib.SFA_DKV_ATOMIC
    assert lib.sfa_bwd(ctypes.byref(b), None, 0, None) == _lib.SFA_E_WORKSPACE


def _valid_pages():
    pg = _lib.KvPages()
    pg.block_table = 0x10000
    pg.bt_sb, pg.max_pages, pg.page_size, pg.num_pages = 2, 2, 4, 4
    return pg


@pytest.mark.parametrize("field,value", [
    ("block_table", None), ("page_size", 3), ("page_size", 0), ("max_pages", 0), ("num_pages", 0),
    ("num_pages", 1 << 30), ("flags", 1), ("max_pages", 1),
])
def test_paged_arguments_are_rejected(field, value):
    lib = _lib.load()
    a = _valid_args()                  # Skv = 8 = max_pages * page_size
    pg = _valid_pages()
    setattr(pg, field, value)
    rc = lib.sfa_fwd_paged(ctypes.byref(a), ctypes.byref(pg), None, 0, None)
    assert rc == _lib.SFA_E_INVALID, field
    assert lib.sfa_last_error()
    assert lib.sfa_fwd_paged_workspace_size(ctypes.byref(a), ctypes.byref(pg)) == 0
    assert lib.sfa_fwd_paged(ctypes.byref(a), None, None, 0, None) == _lib.SFA_E_INVALID


def test_paged_workspace_matches_contiguous_plan():
    lib = _lib.load()
    a = _valid_args()
    a.B, a.Sq, a.Skv, a.Hq, a.Hkv, a.Dqk, a.Dv, a.topk = 64, 1, 65536, 128, 1, 576, 512, 2048
    a.k_ss = a.v_ss = a.k_sh = a.v_sh = 576
    a.k_sb = a.v_sb = 64 * 576          # page stride of a 64-row page pool
    a.q_sh, a.q_ss, a.q_sb = 576, 128 * 576, 128 * 576
    a.o_sh, a.o_ss, a.o_sb = 512, 128 * 512, 128 * 512
    a.v = a.k
    pg = _valid_pages()
    pg.max_pages, pg.page_size, pg.num_pages, pg.bt_sb = 1024, 64, 65536, 1024
    ws = lib.sfa_fwd_paged_workspace_size(ctypes.byref(a), ctypes.byref(pg))
    assert ws > 0
    a.k_sb = a.v_sb = 65536 * 576
    assert ws == lib.sfa_fwd_workspace_size(ctypes.byref(a))



def _d128_bwd_args(B, S, Hq, Hkv, K, mode):
    """Backward arguments of a contiguous bf16 d=128 problem (Sq = Skv = S)."""
    b = _lib.BwdArgs()
    a = b.fwd
    a.dtype = _lib.SFA_DTYPE_BF16
    a.B, a.Sq, a.Skv, a.Hq, a.Hkv, a.Dqk, a.Dv, a.topk = B, S, S, Hq, Hkv, 128, 128, K
    for name in ("q", "k", "v", "idx", "out", "lse"):
        setattr(a, name, 0x10000)
    a.q_sh, a.q_ss, a.q_sb = 128, Hq * 128, S * Hq * 128
    a.o_sh, a.o_ss, a.o_sb = a.q_sh, a.q_ss, a.q_sb
    a.k_sh, a.k_ss, a.k_sb = 128, Hkv * 128, S * Hkv * 128
    a.v_sh, a.v_ss, a.v_sb = a.k_sh, a.k_ss, a.k_sb
    a.i_sh, a.i_ss, a.i_sb = K, Hkv * K, S * Hkv * K
    a.l_sh, a.l_ss, a.l_sb = 1, Hq, S * Hq
    for name in ("dout", "dq", "dk", "dv"):
        setattr(b, name, 0x10000)
    b.do_sh, b.do_ss, b.do_sb = a.q_sh, a.q_ss, a.q_sb
    b.dq_sh, b.dq_ss, b.dq_sb = a.q_sh, a.q_ss, a.q_sb
    b.dk_sh, b.dk_ss, b.dk_sb = a.k_sh, a.k_ss, a.k_sb
    b.dv_sh, b.dv_ss, b.dv_sb = a.k_sh, a.k_ss, a.k_sb
    b.dkv_mode = mode
    return b


def _bwd_ws(B, S, Hq, Hkv, K, mode):
    lib = _lib.load()
    b = _d128_bwd_args(B, S, Hq, Hkv, K, mode)
    return lib.sfa_bwd_workspace_size(ctypes.byref(b))


def test_auto_dkv_scheme_follows_the_cost_rules():
    """AUTO takes the deterministic (CSR) scheme on the GQA training shape,
    and the fp32 atomics where the CSR workspace would exceed 4 GiB (a 64K
    context: its fp32 partials alone are 4.3 GB) or the key range exceeds
    64 x top-k (dense recompute beyond ~32x the selected pairs)."""
    args = (2, 8192, 32, 2, 1024)  # B=2, S=8192, Hq=32, Hkv=2, top-k 1024
    csr, atomic, auto = (_bwd_ws(*args, m) for m in (_lib.SFA_DKV_CSR, _lib.SFA_DKV_ATOMIC, _lib.SFA_DKV_AUTO))
    assert csr > atomic > 0 and auto == csr
    for args in ((1, 65536, 16, 1, 2048), (1, 32768, 16, 1, 256)):
        csr, atomic, auto = (_bwd_ws(*args, m) for m in (_lib.SFA_DKV_CSR, _lib.SFA_DKV_ATOMIC, _lib.SFA_DKV_AUTO))
        assert csr > atomic > 0 and auto == atomic, args
    # at 64K the explicitly requested CSR workspace is the one AUTO avoids
    assert _bwd_ws(1, 65536, 16, 1, 2048, _lib.SFA_DKV_CSR) > (4 << 30)


def test_mla_backward_workspace_holds_two_buffer_sets():
    """The MLA shared-KV backward at S = 32768, top-k 2048: fp32 accumulators
    of the shared rows, delta, then per chunk of queries the P / dS blocks
    (1 MiB per query at 128 heads); the deterministic modes run 1024-query
    chunks and hold two sets of contribution rows and index maps (one
    chunk's reduction reads one set while the next chunk fills the other),
    the atomic mode 2048-query chunks and no set."""
    lib = _lib.load()
    S, K = 32768, 2048

    def ws(mode):
        b = _lib.BwdArgs()
        b.fwd = _mla_prefill_args(S, K)
        b.flags = _lib.SFA_BWD_MERGE_KV
        for name in ("dout", "dq", "dk"):
            setattr(b, name, 0x10000)
        b.do_sh, b.do_ss, b.do_sb = 512, 128 * 512, S * 128 * 512
        b.dq_sh, b.dq_ss, b.dq_sb = 576, 128 * 576, S * 128 * 576
        b.dk_sh, b.dk_ss, b.dk_sb = 576, 576, S * 576
        b.dkv_mode = mode
        return lib.sfa_bwd_workspace_size(ctypes.byref(b))

    acc = S * 576 * 4 + S * 128 * 4           # shared-row accumulators + delta (both 256-aligned here)
    pd = (K // 32) * 2 * 2 * 4 * 512 * 2       # P / dS of one query: 1 MiB
    assert pd == 1 << 20
    words = (S + 2047) // 2048 * 64            # bitmap words per query
    one_set = K * 576 * 2 + words * 6 + K      # contribution rows, bitmap + prefixes, repeat flags
    for mode in (_lib.SFA_DKV_AUTO, _lib.SFA_DKV_CSR):
        assert ws(mode) == acc + 1024 * pd + 2 * 1024 * one_set
    assert 5 << 30 < ws(_lib.SFA_DKV_AUTO) < 6 << 30
    assert ws(_lib.SFA_DKV_ATOMIC) == acc + 2048 * pd


def test_huge_row_strides_leave_the_24_bit_gathers():
    """A K/V row stride of 16 MiB or more cannot go through the kernels whose
    gathers multiply row ids with __umul24: the backward then takes neither
    the CSR scheme nor the MFMA kernels (its workspace is the atomic one)."""
    lib = _lib.load()
    b = _d128_bwd_args(1, 64, 16, 1, 32, _lib.SFA_DKV_AUTO)
    small = lib.sfa_bwd_workspace_size(ctypes.byref(b))
    b.fwd.k_ss = b.fwd.v_ss = 1 << 23  # 16 MiB rows (bf16); Skv = 64 keeps offsets < 2^31
    b.fwd.k_sb = b.fwd.v_sb = 64 << 23
    big = lib.sfa_bwd_workspace_size(ctypes.byref(b))
    assert big < small  # no CSR arrays
    b.dkv_mode = _lib.SFA_DKV_CSR
    for name in ("dout", "dq", "dk", "dv"):
        setattr(b, name, 0x10000)
    assert lib.sfa_bwd(ctypes.byref(b), ctypes.c_void_p(0x10000), 1 << 40, None) == _lib.SFA_E_UNSUPPORTED


def test_noalloc_rejects_plans_beyond_its_scratch():
    """sfa_fwd_noalloc refuses a split-k plan whose partials exceed its
    64 MiB static scratch before touching the device (so this runs without
    a GPU): the MLA decode shape at 8 splits needs 8 x 64 x 128 x 512 bf16."""
    lib = _lib.load()
    a = _valid_args()
    a.B, a.Sq, a.Skv, a.Hq, a.Hkv, a.Dqk, a.Dv, a.topk = 64, 1, 65536, 128, 1, 576, 512, 2048
    a.k_ss = a.v_ss = a.k_sh = a.v_sh = 576
    a.k_sb = a.v_sb = 65536 * 576
    a.q_sh, a.q_ss, a.q_sb = 576, 128 * 576, 128 * 576
    a.o_sh, a.o_ss, a.o_sb = 512, 128 * 512, 128 * 512
    a.v = a.k
    a.num_splits = 8
    need = lib.sfa_fwd_workspace_size(ctypes.byref(a))
    assert need > _lib.SFA_NOALLOC_SCRATCH_BYTES
    assert lib.sfa_fwd_noalloc(ctypes.byref(a), None) == _lib.SFA_E_WORKSPACE
    assert b"static scratch" in lib.sfa_last_error()
    a.topk = 0
    assert lib.sfa_fwd_noalloc(ctypes.byref(a), None) == _lib.SFA_E_INVALID


def test_probe_library_rejects_bad_arguments_without_launching():
    """The measurement-only probe library (bench.py --probe decode_gather)
    builds beside libsfa.so and refuses arguments outside its limits before
    any launch (no GPU needed for these calls)."""
    import os
    path = os.path.join(os.path.dirname(_lib.__file__), "libsfa_probe.so")
    if not os.path.exists(path):
        pytest.skip("libsfa_probe.so is not built (python -m ops_amd.build)")
    lib = ctypes.CDLL(path)
    f = lib.sfa_probe_gather
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                  ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    ok = dict(kv=0x10000, q=0x10000, qr=147456, idx=0x10000, part=0x10000, B=64, Skv=65536, K=2048, s=4, hg=1,
              qb=0, rows=0)
    for bad in (dict(B=0), dict(s=0), dict(K=4096, s=1), dict(Skv=1 << 21), dict(qb=200000), dict(rows=4, part=None),
                dict(hg=-1)):
        a = {**ok, **bad}
        assert f(a["kv"], a["q"], a["qr"], a["idx"], a["part"], a["B"], a["Skv"], a["K"], a["s"], a["hg"], a["qb"],
                 a["rows"], None) == -1, bad
    g = lib.sfa_probe_rowread
    g.restype = ctypes.c_int
    g.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                  ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    ok = dict(kv=0x10000, idx=0x10000, sink=0x10000, B=64, Skv=65536, K=2048, wgs=256, cont=0)
    for bad in (dict(kv=None), dict(sink=None), dict(B=0), dict(wgs=0), dict(idx=None),
                dict(cont=1, Skv=1024)):
        a = {**ok, **bad}
        assert g(a["kv"], a["idx"], a["sink"], a["B"], a["Skv"], a["K"], a["wgs"], a["cont"], None) == -1, bad
