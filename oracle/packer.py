"""Test infrastructure only (imported by tests/, never by the product): a
plain-Python restatement of the reference's training data path, to check the
native loader (autoresearch_amd/csrc/ar_data.cpp) against.

  documents()    prepare.py:256-276 (_document_batches): files in name order,
                 each row group in batches of 128 documents, forever, with the
                 epoch counter incremented after every pass.
  batches()      dataloader_cpu.py:12-58 (make_dataloader_cpu): BOS-aligned
                 best-fit packing of T+1-token rows.
The token-shard reader follows the file layout documented in include/ar_data.h.
"""
from __future__ import annotations

import os

import numpy as np

VAL_SHARD = "shard_06542.tok"


def read_shard(path):
    with open(path, "rb") as f:
        buf = f.read()
    assert buf[:4] == b"ARTK" and np.frombuffer(buf, np.uint32, 1, 4)[0] == 1
    ng, nd, nt = (int(v) for v in np.frombuffer(buf, np.uint64, 3, 8))
    off = 32
    groups = np.frombuffer(buf, np.uint64, ng + 1, off); off += 8 * (ng + 1)
    doc_tokens = np.frombuffer(buf, np.uint64, nd + 1, off); off += 8 * (nd + 1)
    tokens = np.frombuffer(buf, np.int32, nt, off)
    docs = [tokens[int(doc_tokens[d]):int(doc_tokens[d + 1])].tolist() for d in range(nd)]
    return [docs[int(groups[g]):int(groups[g + 1])] for g in range(ng)]


def documents(data_dir, split, tokenizer_batch_size=128):
    names = sorted(n for n in os.listdir(data_dir) if n.endswith(".tok"))
    paths = [os.path.join(data_dir, n) for n in names if (n == VAL_SHARD) == (split == "val")]
    epoch = 1
    while True:
        for p in paths:
            for rg in read_shard(p):
                for i in range(0, len(rg), tokenizer_batch_size):
                    yield rg[i:i + tokenizer_batch_size], epoch
        epoch += 1


def batches(data_dir, split, B, T, buffer_size=1000):
    row_capacity = T + 1
    docs = documents(data_dir, split)
    doc_buffer = []
    epoch = 1
    row_buffer = np.zeros((B, row_capacity), np.int64)
    while True:
        for row_idx in range(B):
            pos = 0
            while pos < row_capacity:
                while len(doc_buffer) < buffer_size:
                    doc_batch, epoch = next(docs)
                    doc_buffer.extend(doc_batch)
                remaining = row_capacity - pos
                best_idx, best_len = -1, 0
                for i, doc in enumerate(doc_buffer):
                    if len(doc) <= remaining and len(doc) > best_len:
                        best_idx, best_len = i, len(doc)
                if best_idx >= 0:
                    doc = doc_buffer.pop(best_idx)
                    row_buffer[row_idx, pos:pos + len(doc)] = doc
                    pos += len(doc)
                else:
                    shortest_idx = min(range(len(doc_buffer)), key=lambda i: len(doc_buffer[i]))
                    doc = doc_buffer.pop(shortest_idx)
                    row_buffer[row_idx, pos:pos + remaining] = doc[:remaining]
                    pos += remaining
        yield row_buffer[:, :-1].copy(), row_buffer[:, 1:].copy(), epoch


def lr_multiplier(progress, warmup=0.0, warmdown=0.5, final_frac=0.0):
    """train.mojo:25-33 with config.mojo:81-83."""
    if progress < warmup:
        return progress / warmup if warmup > 0 else 1.0
    if progress < 1.0 - warmdown:
        return 1.0
    cd = (1.0 - progress) / warmdown
    return cd + (1.0 - cd) * final_frac
