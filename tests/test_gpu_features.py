"""List-feature truncation on the device (``mdl_bag_truncate`` through the
``mdl_hip::bag_truncate`` op): bit-exact against the op's CPU kernel, which
tests/test_features.py pins to the oracle and the reference's golden vectors."""

import json
import sys
import time
from pathlib import Path

import numpy as np
import pyarrow as pa
import pytest
import torch

import mdl_amd  # noqa: F401  (registers the mdl_hip ops)
from mdl_amd.features import bag_csr_arrow
from oracle import oracle as O

pytestmark = pytest.mark.gpu

GOLD = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def announce(*parts):
    print("CASE", *parts, flush=True)
    sys.stdout.flush()


def _inputs(rng, rows, max_len, null_rows=0.1, null_elems=0.1, zeros=False):
    lengths = rng.integers(0, max_len + 1, size=rows)
    offsets = np.zeros(rows + 1, dtype=np.int64)
    np.cumsum(lengths, out=offsets[1:])
    n = int(offsets[-1])
    raw = rng.integers(-(1 << 63), (1 << 63) - 1, size=n, dtype=np.int64, endpoint=True)
    raw[:4] = [-(1 << 63), (1 << 63) - 1, -1, 1][: min(4, n)]
    if zeros and n:
        raw[rng.random(n) < 0.01] = 0
    valid = (rng.random(n) >= null_elems).astype(np.uint8)
    row_valid = (rng.random(rows) >= null_rows).astype(np.uint8)
    return offsets, raw, valid, row_valid


def _run(device, offsets, raw, valid, row_valid, max_length, truncation, bucket, nb, validate=True):
    def t(a, dev, dt=torch.int64):
        return None if a is None else torch.from_numpy(np.asarray(a)).to(dt).to(dev)

    out = []
    for dev in (device, "cpu"):
        res = torch.ops.mdl_hip.bag_truncate(t(raw, dev), t(offsets, dev), t(valid, dev, torch.uint8),
                                             t(row_valid, dev, torch.uint8), max_length, truncation, bucket, nb,
                                             validate)
        out.append([r.cpu() for r in res])
    return out


@pytest.mark.parametrize("bucket,nb", [("none", 0), ("pre_hashed", 1 << 20), ("mod", 1_000_003)])
@pytest.mark.parametrize("truncation", ["head", "tail"])
@pytest.mark.parametrize("max_length", [-1, 0, 3, 32])
def test_bag_truncate_device_equals_cpu_kernel(device, bucket, nb, truncation, max_length):
    announce("bag_truncate", bucket, truncation, max_length)
    rng = np.random.default_rng(100 + max_length)
    offsets, raw, valid, row_valid = _inputs(rng, 3000, 48, zeros=True)
    (gi, gl, go, ge), (ci, cl, co, ce) = _run(device, offsets, raw, valid, row_valid, max_length, truncation,
                                              bucket, nb)
    assert torch.equal(gl, cl) and torch.equal(go, co)
    assert torch.equal(gi, ci)
    assert int(ge[0]) == int(ce[0])


def test_bag_truncate_device_edge_cases(device):
    announce("bag_truncate", "edges")
    rng = np.random.default_rng(7)
    cases = []
    cases.append((np.zeros(1, np.int64), np.zeros(0, np.int64), None, None))  # no rows
    cases.append((np.zeros(5, np.int64), np.zeros(0, np.int64), None, None))  # empty rows, no values
    o, r, v, rv = _inputs(rng, 50, 10)
    cases.append((o, r, v, np.zeros(50, np.uint8)))  # every row null
    cases.append((o + 7, np.concatenate([np.arange(7), r]).astype(np.int64), None, None))  # offsets not from 0
    cases.append((np.array([0, 9, 4, -3, 12], np.int64), np.arange(10, dtype=np.int64), None, None))  # malformed
    for i, (o, r, v, rv) in enumerate(cases):
        for trunc in ("head", "tail"):
            (gi, gl, go, ge), (ci, cl, co, ce) = _run(device, o, r, v, rv, 2, trunc, "mod", 17)
            assert torch.equal(gi, ci) and torch.equal(gl, cl) and torch.equal(go, co), (i, trunc)
            assert int(ge[0]) == int(ce[0]), (i, trunc)


def test_bag_truncate_device_full_batch_matches_oracle(device):
    """A c1-sized bag batch: 50 features x 8192 rows of up to 48 ids, kept to
    the last 32, pre_hashed into 2^20 buckets."""

    announce("bag_truncate", "full batch")
    rng = np.random.default_rng(8)
    offsets, raw, valid, row_valid = _inputs(rng, 50 * 8192, 48)
    raw[raw == 0] = 1
    t0 = time.time()
    (gi, gl, go, ge), _ = _run(device, offsets, raw, valid, row_valid, 32, "tail", "pre_hashed", 1 << 20)
    vals, ok, lengths = O.bag_truncate(offsets, raw, valid, row_valid, 32, "tail")
    ref, _ = O.bucketize_pre_hashed(vals, 1 << 20, ok)
    total = int(lengths.sum())
    assert gl.numpy().tolist() == lengths.tolist()
    assert np.array_equal(gi.numpy()[:total], ref) and not gi.numpy()[total:].any()
    assert int(go[-1]) == total and int(ge[0]) == 0
    announce("bag_truncate", "full batch checked", f"{time.time() - t0:.1f}s", total)


@pytest.mark.parametrize("key", ["bag_head_truncation", "bag_tail_truncation"])
def test_bag_csr_arrow_golden_on_device(device, key):
    g = GOLD[key]
    out = bag_csr_arrow(pa.array(g["rows"], type=pa.list_(pa.int64())), device=device, max_length=g["max_length"],
                        truncation=g["truncation"], bucket="pre_hashed", num_buckets=g["num_buckets"])
    assert out["values"].device.type == "cuda"
    assert out["values"].cpu().tolist() == g["expected_values"]
    assert out["lengths"].cpu().tolist() == g["expected_lengths"]


def test_bag_truncate_opcheck_rocm(device):
    rng = np.random.default_rng(3)
    offsets, raw, valid, row_valid = _inputs(rng, 40, 6)
    raw[raw == 0] = 1
    t = lambda a, dt=torch.int64: torch.from_numpy(a).to(dt).to(device)  # noqa: E731
    args = (t(raw), t(offsets), t(valid, torch.uint8), t(row_valid, torch.uint8), 3, "tail", "pre_hashed", 64, True)
    torch.library.opcheck(torch.ops.mdl_hip.bag_truncate.default, args)


def test_bucket_tensors_on_the_device_equal_the_host(device):
    """``pre_hashed_bucket_tensor`` / ``mod_bucket_tensor`` on ROCm tensors
    (``mdl_bucketize``): the reference's golden columns, and bit-equal to the
    op's CPU kernel (pinned in tests/test_features.py) on 1 M random int64
    hashes with nulls, for both rules."""

    from mdl_amd.features import mod_bucket_tensor, pre_hashed_bucket_tensor

    announce("bucket_tensors")
    g = GOLD["pre_hashed_column_with_nulls"]
    valid = torch.tensor([v is not None for v in g["raw"]], device=device)
    raw = torch.tensor([0 if v is None else v for v in g["raw"]], dtype=torch.int64, device=device)
    assert pre_hashed_bucket_tensor(raw, g["num_buckets"], valid=valid).tolist() == g["expected"]
    zraw = torch.tensor([1, 0], dtype=torch.int64, device=device)
    with pytest.raises(ValueError, match="non-null zero"):
        pre_hashed_bucket_tensor(zraw, 8)
    assert pre_hashed_bucket_tensor(zraw, 8, validate_nonzero=False).tolist() == [2, 1]

    rng = np.random.default_rng(31)
    host = torch.from_numpy(rng.integers(-(1 << 63), (1 << 63) - 1, size=1 << 20, dtype=np.int64, endpoint=True))
    host[:3] = torch.tensor([-(1 << 63), (1 << 63) - 1, 1])
    nulls = torch.from_numpy(rng.random(host.numel()) >= 0.05)
    host_nz = torch.where(host == 0, torch.ones_like(host), host)
    for nb in (8, 1 << 20, 1 << 62):
        want = pre_hashed_bucket_tensor(host_nz, nb, valid=nulls)
        got = pre_hashed_bucket_tensor(host_nz.to(device), nb, valid=nulls.to(device))
        assert torch.equal(got.cpu(), want), nb
    for n in (2, 1_000_000, 999_999_937, (1 << 62) + 1):
        assert torch.equal(mod_bucket_tensor(host.to(device), n).cpu(), mod_bucket_tensor(host, n)), n
