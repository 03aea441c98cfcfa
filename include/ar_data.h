/* ar_data.h -- host-side data and evaluation path of the training driver
 * (libautoresearch_amd.so, C ABI, no GPU calls).
 *
 * The reference tokenizes parquet text with its BPE tokenizer inside Python
 * (prepare.py:_document_batches / Tokenizer.encode, prepare.py:256-297) and
 * packs the token lists into [B, T+1] rows with a BOS-aligned best-fit packer
 * (dataloader_cpu.py:12-58).  The tokenizer and the parquet data are not part
 * of this library: it reads *pre-tokenized* document shards ("token shards"),
 * each document already starting with its BOS token as Tokenizer.encode(...,
 * prepend=bos) produces it, and reproduces the document stream and the packer
 * exactly.
 *
 * Token shard file (little endian):
 *   char     magic[4] = "ARTK";  uint32 version = 1;
 *   uint64   n_groups, n_docs, n_tokens;
 *   uint64   group_docs[n_groups + 1];   row-group boundaries (document index)
 *   uint64   doc_tokens[n_docs + 1];     document boundaries (token index)
 *   int32    tokens[n_tokens];
 * Row groups play the role of parquet row groups: the document stream hands
 * out each group in batches of up to 128 documents (prepare.py:271-276).
 *
 * A data directory holds shard_NNNNN.tok files; files are taken in name
 * order, and shard_06542.tok (VAL_SHARD, prepare.py:42-44) is the validation
 * split, every other shard the training split (prepare.py:256-268).
 *
 * Return codes are the ar_status values of ar_ops.h; ar_last_error() has the
 * message. */
#ifndef AR_DATA_H
#define AR_DATA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ar_loader ar_loader;

/* prepare.py:make_dataloader / dataloader_cpu.py:12-58 for split "train" or
 * "val" of data_dir: B rows of T+1 tokens per batch, buffer_size documents
 * kept in the best-fit pool (1000 in the reference). */
int32_t ar_loader_create(ar_loader** out, const char* data_dir, const char* split, int64_t B, int64_t T,
                         int64_t buffer_size);
/* The next batch (dataloader_cpu.py:31-58): inputs = rows[:, :-1], targets =
 * rows[:, 1:], both host int64 [B*T]; *epoch = the document stream's epoch
 * (1-based) at the time of the last refill. */
int32_t ar_loader_next(ar_loader* loader, int64_t* inputs, int64_t* targets, int64_t* epoch);
int32_t ar_loader_destroy(ar_loader* loader);

/* Write a token shard (the converter a user runs on tokenized data).
 * doc_tokens: n_docs + 1 token offsets; group_docs: n_groups + 1 document
 * offsets (n_groups = 0 writes one group of all documents). */
int32_t ar_shard_write(const char* path, const int32_t* tokens, const uint64_t* doc_tokens, int64_t n_docs,
                       const uint64_t* group_docs, int64_t n_groups);

/* token_bytes (prepare.py:184-195): int32 [V] raw file -> out[V]. */
int32_t ar_token_bytes_load(const char* path, int32_t* out, int64_t vocab_size);

/* evaluate_bpb accumulation (train.mojo:107-118): for each token with
 * 0 <= target < V and token_bytes[target] > 0, *nats += loss, *bytes +=
 * token_bytes[target]. */
int32_t ar_bpb_accumulate(const float* token_loss, const int64_t* targets, const int32_t* token_bytes, int64_t n,
                          int64_t vocab_size, double* nats, double* bytes);

#ifdef __cplusplus
}
#endif

#endif
