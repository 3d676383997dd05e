"""C ABI of libmdl_hip.so without a GPU: exports, struct layout, host-only
entry points and argument validation (no kernel is launched here)."""

import ctypes
import re
import subprocess

import numpy as np
import pytest

from mdl_amd import _lib, ops
from tests.conftest import ROOT

HEADER = ROOT / "include" / "mdl_hip.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mdl_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    lib = _lib.lib()
    names = _declared_functions()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_struct_layout_matches_header(tmp_path):
    probe = tmp_path / "probe.c"
    fields = {
        "mdl_feature": _lib.FEATURE_DTYPE,
        "mdl_chunk": _lib.CHUNK_DTYPE,
        "mdl_table": _lib.TABLE_DTYPE,
        "mdl_update": _lib.UPDATE_DTYPE,
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){"]
    for st, dt in fields.items():
        lines.append(f'printf("{st} size %zu\\n", sizeof({st}));')
        for name in dt.names:
            lines.append(f'printf("{st} {name} %zu\\n", offsetof({st}, {name}));')
    lines.append("return 0;}")
    probe.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", str(probe), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {}
    for line in out:
        if line:
            st, name, val = line.split()
            got[(st, name)] = int(val)
    for st, dt in fields.items():
        assert got[(st, "size")] == dt.itemsize
        for name in dt.names:
            assert got[(st, name)] == dt.fields[name][1], (st, name)


def test_plan_chunks_host_helper():
    lib = _lib.lib()
    feats = np.zeros(3, dtype=_lib.FEATURE_DTYPE)
    feats["pooling"] = [_lib.MDL_POOL_MEAN, _lib.MDL_POOL_NONE, _lib.MDL_POOL_SUM]
    feats["num_bags"] = [8192, 0, 1000]
    feats["num_ids"] = [8192 * 16, 1500, 1000]
    n = lib.mdl_plan_chunks(feats.ctypes.data, 3, 512, None, 0)
    chunks = np.zeros(n, dtype=_lib.CHUNK_DTYPE)
    assert lib.mdl_plan_chunks(feats.ctypes.data, 3, 512, chunks.ctypes.data, n) == n
    f0 = chunks[chunks["feature"] == 0]
    assert (f0["count"] == 32).all() and f0["count"].sum() == 8192  # 32 bags x ~16 ids
    assert f0["first"].tolist() == list(range(0, 8192, 32))
    f1 = chunks[chunks["feature"] == 1]
    assert f1["count"].tolist() == [512, 512, 476] and f1["first"].tolist() == [0, 512, 1024]
    f2 = chunks[chunks["feature"] == 2]
    assert f2["count"].max() == 256 and f2["count"].sum() == 1000  # bag cap 256
    assert lib.mdl_plan_chunks(feats.ctypes.data, 3, 0, None, 0) == _lib.MDL_OK - 1  # MDL_ERR_INVALID


def test_invalid_arguments_fail_before_any_launch():
    lib = _lib.lib()
    rc = lib.mdl_bucketize(None, None, 4, 6, _lib.MDL_BUCKET_PRE_HASHED, 1, None, None, None)
    assert rc == -1 and b"power of two" in lib.mdl_last_error()
    rc = lib.mdl_bucketize(None, None, 4, 1, _lib.MDL_BUCKET_MOD, 0, None, None, None)
    assert rc == -1 and b"num_buckets > 1" in lib.mdl_last_error()
    rc = lib.mdl_sort_pairs(None, None, None, None, 10, 40, None, 0, None, None)
    assert rc == -1 and b"key_bits" in lib.mdl_last_error()
    rc = lib.mdl_sort_pairs(None, None, None, None, 1 << 33, 8, None, 0, None, None)
    assert rc == -4
    rc = lib.mdl_backward_adagrad(None, 0, None, 0, 8, None, None, 10, None, 8, None, 0.1, 1e-8, None, None, 0, 0,
                                  None)
    assert rc == -1 and b"table" in lib.mdl_last_error()
    rc = lib.mdl_backward_apply(None, 0, None, 1, 0, None, None, 10, 8, None, 0.1, 1e-8, None, None, 0, 0, None)
    assert rc == -1 and b"max_dim" in lib.mdl_last_error()
    # rows of any width pass validation (wide ones are walked in column blocks): no workspace is what fails
    rc = lib.mdl_backward_apply(None, 0, None, 1, 600, None, None, 10, 8, None, 0.1, 1e-8, None, None, 0, 0, None)
    assert rc == -3
    rc = lib.mdl_forward(None, 0, None, 1, None, -1, None, None, None, None, 0, None, None, 0, None)
    assert rc == -1
    rc = lib.mdl_rowwise_adagrad(None, _lib.MDL_F32, 10, 4, 4, None, None, 3, None, _lib.MDL_BF16, 4, 0.1,
                                 1e-8, None, None)
    assert rc == -1  # null pointers
    # zero-sized work is a no-op success without touching the device
    assert lib.mdl_forward(None, 0, None, 0, None, 0, None, None, None, None, 0, None, None, 0, None) == 0
    assert lib.mdl_rowwise_adagrad(None, 0, 0, 4, 4, None, None, 0, None, 0, 4, 0.1, 1e-8, None, None) == 0


def test_workspace_queries_are_monotone():
    """A workspace sized for the largest call serves every smaller one, also
    across the sizes where the sort tiles and the backward chunks change
    (about 0.5 M to 2.2 M entries)."""

    lib = _lib.lib()
    prev = (0, 0, 0)
    for n in range(0, 3_000_000, 4099):
        cur = (lib.mdl_backward_workspace_bytes(n, 8, 64), lib.mdl_sort_workspace_bytes(n),
               lib.mdl_unique_workspace_bytes(n))
        assert all(c >= p for c, p in zip(cur, prev)), n
        prev = cur
    for n in (524_287, 557_055, 1_048_575, 1_572_863, 2_097_151):  # where tiles and chunks change
        for f in (lambda m: lib.mdl_backward_workspace_bytes(m, 8, 64), lib.mdl_sort_workspace_bytes,
                  lib.mdl_unique_workspace_bytes):
            assert f(n) <= f(n + 1) <= f(n + 4096), n
    a = lib.mdl_backward_workspace_bytes(1000, 4, 64)
    b = lib.mdl_backward_workspace_bytes(100000, 4, 64)
    c = lib.mdl_backward_workspace_bytes(100000, 200, 128)
    assert 0 < a < b < c
    assert lib.mdl_sort_workspace_bytes(1 << 20) >= 256 * 256 * 4
    assert lib.mdl_unique_workspace_bytes(1000) > 16 * 1000


def test_class_masks_follow_dtype_and_alignment():
    lib = _lib.lib()
    feats = np.zeros(3, dtype=_lib.FEATURE_DTYPE)
    feats["wdtype"] = [_lib.MDL_F32, _lib.MDL_BF16, _lib.MDL_BF16]
    feats["odtype"] = [_lib.MDL_F32, _lib.MDL_BF16, _lib.MDL_F32]
    feats["dim"] = [64, 64, 12]           # bf16 x 12 = 24 bytes: not 16-byte rows
    feats["out_stride"] = [64, 64, 12]
    feats["weight"] = [256, 512, 1024]
    feats["out"] = [4096, 8192, 8196]
    m = lib.mdl_feature_classes(feats.ctypes.data, 3)
    # variant = 3 * class + log2(C / 4): fp32 x 64 moves 8 per lane (class 0),
    # bf16 x 64 8 per lane (class 2), unaligned bf16 -> fp32 rows 1 (class 5)
    assert m == (1 << (3 * 0 + 1)) | (1 << (3 * 2 + 1)) | (1 << (3 * 5))
    tables = np.zeros(2, dtype=_lib.TABLE_DTYPE)
    tables["wdtype"] = [_lib.MDL_F32, _lib.MDL_BF16]
    tables["gdtype"] = [_lib.MDL_F32, _lib.MDL_BF16]
    tables["dim"] = [3, 32]
    tables["weight"] = [256, 512]
    # fp32 x 3 is unaligned (class 1); bf16 x 32: four lanes of 8 cover it (class 2, C = 8)
    assert lib.mdl_table_classes(tables.ctypes.data, 2) == (1 << (3 * 1)) | (1 << (3 * 2 + 1))


@pytest.mark.parametrize("dim,esize,vec,expect", [
    (16, 4, True, 4), (32, 4, True, 8), (64, 4, True, 8), (128, 4, True, 8), (24, 4, True, 8),
    (40, 4, True, 8), (300, 4, True, 4), (8, 2, True, 8), (64, 2, True, 8), (24, 2, True, 8), (3, 4, False, 1),
])
def test_lane_width_rule(dim, esize, vec, expect):
    # C divides dim, so a lane's elements lie wholly inside the row
    c = ops.lane_elems(dim, esize, vec)
    assert c == expect and dim % c == 0


def test_lane_width_rule_matches_the_library():
    """The host rule and the library's variant of a table agree for every dim
    and dtype, rows wider than 64 lanes cover included (the reduce walks them
    in column blocks, so no mask carries the reserved unsupported bit)."""
    lib = _lib.lib()
    tables = np.zeros(1, dtype=_lib.TABLE_DTYPE)
    for wd, esize in ((_lib.MDL_F32, 4), (_lib.MDL_BF16, 2)):
        for dim in list(range(1, 300)) + [520, 600, 1024, 1030]:
            tables["wdtype"] = wd
            tables["gdtype"] = wd
            tables["dim"] = dim
            tables["weight"] = 4096
            m = lib.mdl_table_classes(tables.ctypes.data, 1)
            vec = (dim * esize) % 16 == 0
            c = ops.lane_elems(dim, esize, vec)
            cls = (0 if wd == _lib.MDL_F32 else 2) + (0 if vec else 1)
            w = 0 if c == 1 else {4: 0, 8: 1, 16: 2}[c]
            assert m == 1 << (3 * cls + w), (wd, dim)


@pytest.mark.parametrize("dim,dtype", [(66, "f32"), (100, "bf16"), (300, "f32"), (600, "f32")])
def test_wide_rows_have_a_class_and_the_reserved_bit_is_refused(dim, dtype):
    """Rows wider than 64 lanes cover get their table's ordinary class (the
    reduce walks them in column blocks); a mask carrying the reserved
    MDL_CLASSES_UNSUPPORTED bit is refused by every reducing call before it
    launches anything."""

    lib = _lib.lib()
    tables = np.zeros(1, dtype=_lib.TABLE_DTYPE)
    code = _lib.MDL_F32 if dtype == "f32" else _lib.MDL_BF16
    tables["wdtype"] = code
    tables["gdtype"] = code
    tables["dim"] = dim
    tables["weight"] = 4096
    m = lib.mdl_table_classes(tables.ctypes.data, 1)
    assert m and not m & _lib.MDL_CLASSES_UNSUPPORTED
    m |= _lib.MDL_CLASSES_UNSUPPORTED
    for call in (
        lambda: lib.mdl_backward_apply(None, 1, None, 1, 512, None, None, 10, 8, None, 0.1, 1e-8, None, None, 0,
                                       m, None),
        lambda: lib.mdl_backward_sumsq(None, 1, None, 1, 512, None, None, 10, 8, None, None, None, 0, m, None),
        lambda: lib.mdl_backward_coalesce(None, 1, None, 1, 512, None, None, 10, 8, None, None, None, None, None, 0,
                                          m, None),
        lambda: lib.mdl_backward_adagrad(None, 1, None, 1, 512, None, None, 10, None, 8, None, 0.1, 1e-8, None, None,
                                         0, m, None),
    ):
        assert call() == -4 and b"reserved" in lib.mdl_last_error()


def test_abi_version_matches_binding():
    assert _lib.lib().mdl_abi_version() == _lib.ABI_VERSION


def test_bag_truncate_refuses_bad_arguments_before_any_launch():
    lib = _lib.lib()
    ws_bytes = lib.mdl_bag_truncate_workspace_bytes(4)
    assert ws_bytes >= lib.mdl_offsets_workspace_bytes(4) + 4 * 8
    p = 4096  # never dereferenced: every call below fails its checks first

    def call(rows=4, n_in=8, max_length=3, trunc=_lib.MDL_TRUNCATE_TAIL, mode=_lib.MDL_BUCKET_NONE, buckets=0,
             cap=8, ws=ws_bytes, out_offsets=p):
        return lib.mdl_bag_truncate(p, None, rows, p, None, n_in, max_length, trunc, mode, buckets, 1, p,
                                    out_offsets, p, cap, None, p, ws, None)

    assert call(rows=-1) == -1 and b"negative" in lib.mdl_last_error()
    assert call(cap=-1) == -1
    assert call(trunc=7) == -1 and b"head or tail" in lib.mdl_last_error()
    assert call(mode=9) == -1 and b"unknown bucketing mode" in lib.mdl_last_error()
    assert call(mode=_lib.MDL_BUCKET_PRE_HASHED, buckets=6) == -1 and b"power of two" in lib.mdl_last_error()
    assert call(mode=_lib.MDL_BUCKET_MOD, buckets=1) == -1
    assert call(out_offsets=None) == -1 and b"null pointer" in lib.mdl_last_error()
    assert call(ws=ws_bytes - 1) != 0 and b"workspace" in lib.mdl_last_error()
