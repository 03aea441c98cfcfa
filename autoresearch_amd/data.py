"""Python view of the training driver's data path (include/ar_data.h).

write_shard / write_token_bytes produce the files the native loader reads;
Loader wraps ar_loader_* (the BOS-aligned best-fit packer of the reference's
dataloader_cpu.py:12-58 over the document stream of prepare.py:256-276).
"""
from __future__ import annotations

import ctypes as ct

import numpy as np

from ._lib import check, load

VAL_SHARD = "shard_06542.tok"  # prepare.py:42-44 (pinned validation shard)


def write_shard(path: str, docs, groups=None) -> None:
    """Write a token shard.  docs: sequence of 1-D int token arrays, each
    starting with its BOS token (Tokenizer.encode(..., prepend=bos));
    groups: sizes of the row groups (sum = len(docs)); one group if None."""
    lens = np.array([len(d) for d in docs], dtype=np.uint64)
    doc_tokens = np.zeros(len(docs) + 1, dtype=np.uint64)
    np.cumsum(lens, out=doc_tokens[1:])
    tokens = np.ascontiguousarray(np.concatenate([np.asarray(d, dtype=np.int32) for d in docs])
                                  if len(docs) else np.zeros(0, np.int32))
    if groups is None:
        gd, ng = None, 0
    else:
        gd = np.zeros(len(groups) + 1, dtype=np.uint64)
        np.cumsum(np.asarray(groups, dtype=np.uint64), out=gd[1:])
        ng = len(groups)
    check(load().ar_shard_write(path.encode(), tokens.ctypes.data, doc_tokens.ctypes.data, len(docs),
                                None if gd is None else gd.ctypes.data, ng), "shard_write")


def write_token_bytes(path: str, token_bytes) -> None:
    """token_bytes (prepare.py:184-195) as the int32 [V] file the driver reads."""
    np.asarray(token_bytes, dtype=np.int32).tofile(path)


class Loader:
    """prepare.make_dataloader semantics for one split of a token-shard directory."""

    def __init__(self, data_dir: str, split: str, B: int, T: int, buffer_size: int = 1000):
        self.B, self.T = B, T
        self._h = ct.c_void_p()
        check(load().ar_loader_create(ct.byref(self._h), data_dir.encode(), split.encode(), B, T, buffer_size),
              "loader_create")

    def next(self):
        x = np.empty((self.B, self.T), np.int64)
        y = np.empty((self.B, self.T), np.int64)
        e = ct.c_int64()
        check(load().ar_loader_next(self._h, x.ctypes.data, y.ctypes.data, ct.byref(e)), "loader_next")
        return x, y, e.value

    def close(self):
        if self._h:
            load().ar_loader_destroy(self._h)
            self._h = ct.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def bpb_accumulate(token_loss, targets, token_bytes):
    """(nats, bytes) sums of evaluate_bpb (train.mojo:107-118)."""
    tl = np.ascontiguousarray(token_loss, dtype=np.float32)
    tg = np.ascontiguousarray(targets, dtype=np.int64)
    tb = np.ascontiguousarray(token_bytes, dtype=np.int32)
    nats, nb = ct.c_double(0.0), ct.c_double(0.0)
    check(load().ar_bpb_accumulate(tl.ctypes.data, tg.ctypes.data, tb.ctypes.data, tl.size, tb.size,
                                   ct.byref(nats), ct.byref(nb)), "bpb_accumulate")
    return nats.value, nb.value
