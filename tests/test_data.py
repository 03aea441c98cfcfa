"""Training-driver data path (include/ar_data.h) against the Python
restatement of the reference's packer (oracle/packer.py): bit-exact batches
and epochs for both splits, row-group batching, buffer sizes that force both
the best-fit and the crop branch, and the BPB sums.  Host code only: these
run without a GPU."""
import os

import numpy as np
import pytest

from oracle import packer


def _docs(rng, n, V=500, lo=1, hi=300):
    out = []
    for _ in range(n):
        L = int(rng.integers(lo, hi))
        d = rng.integers(4, V, L).astype(np.int32)
        d[0] = 1  # BOS
        out.append(d)
    return out


@pytest.fixture
def shard_dir(tmp_path):
    from autoresearch_amd import data
    rng = np.random.default_rng(7)
    # three training shards (one with several row groups, one with a group of
    # more than 128 documents) and the pinned validation shard
    data.write_shard(str(tmp_path / "shard_00000.tok"), _docs(rng, 40))
    data.write_shard(str(tmp_path / "shard_00001.tok"), _docs(rng, 300, hi=900), groups=[100, 0, 170, 30])
    data.write_shard(str(tmp_path / "shard_00007.tok"), _docs(rng, 5, lo=2000, hi=3000))
    data.write_shard(str(tmp_path / packer.VAL_SHARD), _docs(rng, 60), groups=[30, 30])
    return str(tmp_path)


@pytest.mark.parametrize("split,B,T,buf,n", [("train", 3, 64, 20, 40), ("train", 2, 512, 1000, 12),
                                             ("train", 1, 1024, 7, 30), ("val", 4, 128, 50, 20)])
def test_loader_matches_reference_packer(shard_dir, split, B, T, buf, n):
    from autoresearch_amd import data
    ld = data.Loader(shard_dir, split, B, T, buf)
    ref = packer.batches(shard_dir, split, B, T, buf)
    epochs = set()
    for i in range(n):
        x, y, e = ld.next()
        rx, ry, re_ = next(ref)
        np.testing.assert_array_equal(x, rx, err_msg=f"batch {i}")
        np.testing.assert_array_equal(y, ry, err_msg=f"batch {i}")
        assert e == re_, (i, e, re_)
        # targets are the inputs shifted by one inside each packed row
        np.testing.assert_array_equal(x[:, 1:], y[:, :-1])
        epochs.add(e)
    ld.close()
    if split == "train" and buf == 1000:
        assert len(epochs) > 1  # the stream wrapped around


def test_rows_start_with_bos_and_splits_are_disjoint(shard_dir):
    """BOS-aligned: every row starts at a document start (dataloader_cpu.py:34);
    the val stream only reads shard_06542 and train never does."""
    from autoresearch_amd import data
    for split in ("train", "val"):
        x, _, _ = data.Loader(shard_dir, split, 8, 128, 1000).next()
        assert np.all(x[:, 0] == 1)
    val_docs = [d for g in packer.read_shard(os.path.join(shard_dir, packer.VAL_SHARD)) for d in g]
    train_first = next(packer.documents(shard_dir, "train"))[0]
    assert all(not np.array_equal(train_first[0], v) for v in val_docs[:5])


def test_document_stream_batches_of_128(shard_dir):
    """prepare.py:271-276: a row group of 170 documents is handed out as 128 + 42."""
    sizes = []
    for batch, epoch in packer.documents(shard_dir, "train"):
        if epoch > 1:
            break
        sizes.append(len(batch))
    assert sizes == [40, 100, 128, 42, 30, 5]


def test_loader_errors(tmp_path):
    from autoresearch_amd import data
    from autoresearch_amd._lib import ArError
    with pytest.raises(ArError):
        data.Loader(str(tmp_path / "missing"), "train", 1, 8)
    with pytest.raises(ArError):
        data.Loader(str(tmp_path), "train", 1, 8)  # no shards
    with pytest.raises(ArError):
        data.Loader(str(tmp_path), "test", 1, 8)
    (tmp_path / "shard_00000.tok").write_bytes(b"XXXX" + b"\0" * 64)
    ld = data.Loader(str(tmp_path), "train", 1, 8)
    with pytest.raises(ArError, match="bad header"):
        ld.next()
    # empty documents are rejected (every tokenized document holds its BOS)
    data.write_shard(str(tmp_path / "shard_00000.tok"), [np.array([1, 5], np.int32), np.zeros(0, np.int32)])
    with pytest.raises(ArError, match="empty"):
        data.Loader(str(tmp_path), "train", 1, 8).next()


def test_bpb_accumulate_closed_form():
    """train.mojo:107-118: nats over tokens whose target is in range and has
    a positive byte length; bytes = their byte lengths."""
    from autoresearch_amd import data
    rng = np.random.default_rng(3)
    V, n = 50, 1000
    tb = rng.integers(0, 6, V).astype(np.int32)  # some special tokens have 0 bytes
    loss = rng.random(n).astype(np.float32) * 5
    tg = rng.integers(-3, V + 3, n).astype(np.int64)  # ignored (-1) and out-of-range targets too
    nats, nb = data.bpb_accumulate(loss, tg, tb)
    keep = (tg >= 0) & (tg < V)
    keep[keep] &= tb[tg[keep]] > 0
    assert nb == float(tb[tg[keep]].sum())
    assert abs(nats - float(loss[keep].astype(np.float64).sum())) <= 1e-9 * max(1.0, nats)
    assert keep.sum() < n  # both exclusions were exercised


def test_token_bytes_roundtrip(tmp_path):
    from autoresearch_amd import data
    from autoresearch_amd._lib import ArError, check, load
    tb = np.arange(17, dtype=np.int32) % 5
    p = str(tmp_path / "token_bytes.bin")
    data.write_token_bytes(p, tb)
    out = np.zeros(17, np.int32)
    check(load().ar_token_bytes_load(p.encode(), out.ctypes.data, 17))
    np.testing.assert_array_equal(out, tb)
    with pytest.raises(ArError):
        check(load().ar_token_bytes_load(p.encode(), np.zeros(40, np.int32).ctypes.data, 40))
