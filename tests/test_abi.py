"""The C-ABI library loads without a GPU and exports every entry point include/mi355moe.h declares; argument
validation fails cleanly before any device work."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "include", "mi355moe.h")


def declared():
    src = open(HDR).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(mm_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_entry_points():
    names = declared()
    for must in ("mm_split", "mm_combine_host", "mm_permute", "mm_combine", "mm_expert_gemv", "mm_router_topk"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from mi355moe import _lib
    L = _lib.load()
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (mm_[a-z0-9_]+)$", out, flags=re.M))
    for name in declared():
        assert name in exported, name
        assert getattr(L, name) is not None
        assert name in _lib.EXPORTS, name


def test_argument_errors_without_device_work():
    from mi355moe import _lib
    L = _lib.load()
    assert L.mm_version() == 100
    rc = L.mm_split(None, None, None, 32, 4, 4096, 2000, None, None, None, None, None, None, None, 0, None, None, None,
                    None, None, None, None, None, None)
    assert rc == -1 and b"E <= 1024" in L.mm_last_error()
    rc = L.mm_permute(None, None, 10, 8, 0, None, None, None, None, None, None, None, None, None, 0, None)
    assert rc == -1
    rc = L.mm_expert_gemv(None, None, 0, 0, 1, 1, 1, None, None, None, None, None, 1, None, None, 0, 31, None)
    assert rc == -1 and b"incomplete layer" in L.mm_last_error()
    with pytest.raises(RuntimeError, match="mm_combine"):
        _lib.call("mm_combine", None, None, None, None, 1, 1, 4096, 8, 0, None)
    assert L.mm_permute_workspace(100, 384) == 0 and L.mm_permute_workspace(131072, 384) > 0
    # transformed gate/up inputs, 8 K parts of gate/up partial sums, the down input, 4 K parts of down partials
    assert L.mm_gemv_workspace(36, 385, 4096, 2048) >= (36 * 2 * 4096 * 2 + 8 * 36 * 2 * 2048 * 4 + 36 * 2048 * 2
                                                        + 4 * 36 * 4096 * 4)
    assert L.mm_gemv_workspace(0, 385, 4096, 2048) == 0


def test_expert_seed_matches_oracle():
    import oracle as O
    from mi355moe import _lib
    L = _lib.load()
    for ls, e in ((1000, 0), (1039, 384), (2**40 + 3, 17)):
        assert L.mm_expert_seed(ls, e) == O.expert_seed(ls, e)
