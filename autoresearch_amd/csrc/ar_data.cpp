// ar_data.cpp -- the training driver's host data path (C ABI in
// include/ar_data.h): token-shard document stream, the BOS-aligned best-fit
// packer of the reference's dataloader, token_bytes and the BPB sums.
//
// Host code only (no HIP); it is linked into libautoresearch_amd.so.
#include <dirent.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/ar_data.h"
#include "../../include/ar_ops.h"

namespace ar {
int32_t set_error(int32_t code, const char* fmt, ...);
}

namespace {

constexpr int kDocBatch = 128;                   // tokenizer_batch_size, prepare.py:256
constexpr const char* kValShard = "shard_06542.tok";  // VAL_SHARD, prepare.py:42-44

struct Shard {
    std::vector<uint64_t> group_docs, doc_tokens;
    std::vector<int32_t> tokens;
};

bool read_all(FILE* f, void* p, size_t n) { return n == 0 || fread(p, 1, n, f) == n; }

int32_t load_shard(const std::string& path, Shard& s) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return ar::set_error(AR_EINVAL, "token shard %s: cannot open", path.c_str());
    char magic[4];
    uint32_t version = 0;
    uint64_t ng = 0, nd = 0, nt = 0;
    bool ok = read_all(f, magic, 4) && memcmp(magic, "ARTK", 4) == 0 && read_all(f, &version, 4) && version == 1 &&
              read_all(f, &ng, 8) && read_all(f, &nd, 8) && read_all(f, &nt, 8) && ng <= nd + 1 &&
              nd < (uint64_t)1 << 40 && nt < (uint64_t)1 << 40;
    if (ok) {
        s.group_docs.resize(ng + 1);
        s.doc_tokens.resize(nd + 1);
        s.tokens.resize(nt);
        ok = read_all(f, s.group_docs.data(), (ng + 1) * 8) && read_all(f, s.doc_tokens.data(), (nd + 1) * 8) &&
             read_all(f, s.tokens.data(), nt * 4);
    }
    fclose(f);
    if (!ok) return ar::set_error(AR_EINVAL, "token shard %s: bad header or truncated", path.c_str());
    if (s.group_docs[0] != 0 || s.group_docs[ng] != nd || s.doc_tokens[0] != 0 || s.doc_tokens[nd] != nt)
        return ar::set_error(AR_EINVAL, "token shard %s: inconsistent offsets", path.c_str());
    for (uint64_t g = 0; g < ng; ++g)
        if (s.group_docs[g] > s.group_docs[g + 1])
            return ar::set_error(AR_EINVAL, "token shard %s: decreasing group offsets", path.c_str());
    for (uint64_t d = 0; d < nd; ++d)
        if (s.doc_tokens[d] >= s.doc_tokens[d + 1])  // every document holds at least its BOS token
            return ar::set_error(AR_EINVAL, "token shard %s: empty or decreasing document %llu", path.c_str(),
                                 (unsigned long long)d);
    return AR_OK;
}

// prepare.py:256-276 (_document_batches): shards in order, each row group in
// batches of up to kDocBatch documents, forever; epoch counts passes.
struct DocStream {
    std::vector<std::string> paths;
    size_t file = 0;
    uint64_t group = 0, doc = 0;  // next document of the current group
    int64_t epoch = 1;
    Shard cur;
    bool loaded = false;

    int32_t next_batch(std::vector<std::vector<int32_t>>& out, int64_t& batch_epoch) {
        for (size_t guard = 0;; ++guard) {
            if (!loaded) {
                const int32_t r = load_shard(paths[file], cur);
                if (r) return r;
                loaded = true;
                group = 0;
                doc = cur.group_docs.empty() ? 0 : cur.group_docs[0];
            }
            const uint64_t ng = cur.group_docs.size() - 1;
            while (group < ng && doc >= cur.group_docs[group + 1]) {
                ++group;
                if (group < ng) doc = cur.group_docs[group];
            }
            if (group < ng) {
                const uint64_t end = std::min(cur.group_docs[group + 1], doc + (uint64_t)kDocBatch);
                for (uint64_t d = doc; d < end; ++d)
                    out.emplace_back(cur.tokens.begin() + (int64_t)cur.doc_tokens[d],
                                     cur.tokens.begin() + (int64_t)cur.doc_tokens[d + 1]);
                doc = end;
                batch_epoch = epoch;
                return AR_OK;
            }
            // next shard (and epoch after the last one)
            loaded = false;
            if (++file == paths.size()) {
                file = 0;
                ++epoch;
            }
            if (guard > 4 * paths.size() + 4)
                return ar::set_error(AR_EINVAL, "token shards hold no documents");
        }
    }
};

}  // namespace

struct ar_loader {
    DocStream stream;
    int64_t B = 0, T = 0, buffer_size = 0, epoch = 1;
    std::vector<std::vector<int32_t>> pool;  // doc_buffer
    std::vector<int64_t> rows;               // row_buffer [B, T+1]
};

extern "C" int32_t ar_loader_create(ar_loader** out, const char* data_dir, const char* split, int64_t B, int64_t T,
                                    int64_t buffer_size) {
    if (!out || !data_dir || !split) return ar::set_error(AR_EINVAL, "loader_create: null pointer");
    const bool train = strcmp(split, "train") == 0, val = strcmp(split, "val") == 0;
    if (!train && !val) return ar::set_error(AR_EINVAL, "loader_create: split must be \"train\" or \"val\"");
    if (B <= 0 || T <= 0 || buffer_size <= 0) return ar::set_error(AR_EINVAL, "loader_create: bad B, T or buffer");
    DIR* d = opendir(data_dir);
    if (!d) return ar::set_error(AR_EINVAL, "loader_create: cannot open %s", data_dir);
    std::vector<std::string> names;
    while (dirent* e = readdir(d)) {
        const std::string n = e->d_name;
        if (n.size() > 4 && n.compare(n.size() - 4, 4, ".tok") == 0) names.push_back(n);
    }
    closedir(d);
    std::sort(names.begin(), names.end());
    ar_loader* l = new ar_loader();
    for (const std::string& n : names)
        if ((n == kValShard) == val) l->stream.paths.push_back(std::string(data_dir) + "/" + n);
    if (l->stream.paths.empty()) {
        delete l;
        return ar::set_error(AR_EINVAL, "loader_create: no %s token shards in %s", split, data_dir);
    }
    l->B = B;
    l->T = T;
    l->buffer_size = buffer_size;
    l->rows.assign((size_t)(B * (T + 1)), 0);
    *out = l;
    return AR_OK;
}

// dataloader_cpu.py:31-58
extern "C" int32_t ar_loader_next(ar_loader* l, int64_t* inputs, int64_t* targets, int64_t* epoch) {
    if (!l || !inputs || !targets) return ar::set_error(AR_EINVAL, "loader_next: null pointer");
    const int64_t cap = l->T + 1;
    for (int64_t row = 0; row < l->B; ++row) {
        int64_t* dst = l->rows.data() + row * cap;
        int64_t pos = 0;
        while (pos < cap) {
            while ((int64_t)l->pool.size() < l->buffer_size) {
                const int32_t r = l->stream.next_batch(l->pool, l->epoch);
                if (r) return r;
            }
            const int64_t remaining = cap - pos;
            // largest document that fits entirely (first one on ties)
            int64_t best = -1, best_len = 0;
            for (size_t i = 0; i < l->pool.size(); ++i) {
                const int64_t n = (int64_t)l->pool[i].size();
                if (n <= remaining && n > best_len) {
                    best = (int64_t)i;
                    best_len = n;
                }
            }
            if (best >= 0) {
                const std::vector<int32_t>& doc = l->pool[best];
                for (int64_t j = 0; j < best_len; ++j) dst[pos + j] = doc[j];
                pos += best_len;
                l->pool.erase(l->pool.begin() + best);
            } else {
                // none fits: crop the shortest (first one on ties) to fill the row
                size_t s = 0;
                for (size_t i = 1; i < l->pool.size(); ++i)
                    if (l->pool[i].size() < l->pool[s].size()) s = i;
                const std::vector<int32_t>& doc = l->pool[s];
                for (int64_t j = 0; j < remaining; ++j) dst[pos + j] = doc[j];
                pos += remaining;
                l->pool.erase(l->pool.begin() + s);
            }
        }
        for (int64_t t = 0; t < l->T; ++t) {
            inputs[row * l->T + t] = dst[t];
            targets[row * l->T + t] = dst[t + 1];
        }
    }
    if (epoch) *epoch = l->epoch;
    return AR_OK;
}

extern "C" int32_t ar_loader_destroy(ar_loader* l) {
    delete l;
    return AR_OK;
}

extern "C" int32_t ar_shard_write(const char* path, const int32_t* tokens, const uint64_t* doc_tokens, int64_t n_docs,
                                  const uint64_t* group_docs, int64_t n_groups) {
    if (!path || !doc_tokens || n_docs < 0 || n_groups < 0 || (n_groups > 0 && !group_docs))
        return ar::set_error(AR_EINVAL, "shard_write: bad arguments");
    const uint64_t nt = doc_tokens[n_docs];
    if (nt > 0 && !tokens) return ar::set_error(AR_EINVAL, "shard_write: null tokens");
    std::vector<uint64_t> groups;
    if (n_groups == 0) groups = {0, (uint64_t)n_docs};
    else groups.assign(group_docs, group_docs + n_groups + 1);
    FILE* f = fopen(path, "wb");
    if (!f) return ar::set_error(AR_EINVAL, "shard_write: cannot create %s", path);
    const uint32_t version = 1;
    const uint64_t ng = groups.size() - 1, nd = (uint64_t)n_docs;
    bool ok = fwrite("ARTK", 1, 4, f) == 4 && fwrite(&version, 4, 1, f) == 1 && fwrite(&ng, 8, 1, f) == 1 &&
              fwrite(&nd, 8, 1, f) == 1 && fwrite(&nt, 8, 1, f) == 1 &&
              fwrite(groups.data(), 8, groups.size(), f) == groups.size() &&
              fwrite(doc_tokens, 8, nd + 1, f) == nd + 1 && (nt == 0 || fwrite(tokens, 4, nt, f) == nt);
    ok = (fclose(f) == 0) && ok;
    return ok ? AR_OK : ar::set_error(AR_EINVAL, "shard_write: write to %s failed", path);
}

extern "C" int32_t ar_token_bytes_load(const char* path, int32_t* out, int64_t vocab_size) {
    if (!path || !out || vocab_size <= 0) return ar::set_error(AR_EINVAL, "token_bytes_load: bad arguments");
    FILE* f = fopen(path, "rb");
    if (!f) return ar::set_error(AR_EINVAL, "token_bytes_load: cannot open %s", path);
    const bool ok = fread(out, 4, (size_t)vocab_size, f) == (size_t)vocab_size;
    fclose(f);
    return ok ? AR_OK : ar::set_error(AR_EINVAL, "token_bytes_load: %s holds fewer than %lld entries", path,
                                      (long long)vocab_size);
}

// train.mojo:107-118
extern "C" int32_t ar_bpb_accumulate(const float* token_loss, const int64_t* targets, const int32_t* token_bytes,
                                     int64_t n, int64_t vocab_size, double* nats, double* bytes) {
    if (!token_loss || !targets || !token_bytes || !nats || !bytes)
        return ar::set_error(AR_EINVAL, "bpb_accumulate: null pointer");
    if (n < 0 || vocab_size < 0) return ar::set_error(AR_EINVAL, "bpb_accumulate: negative count");
    for (int64_t i = 0; i < n; ++i) {
        const int64_t t = targets[i];
        if (t >= 0 && t < vocab_size) {
            const int32_t nb = token_bytes[t];
            if (nb > 0) {
                *nats += (double)token_loss[i];
                *bytes += (double)nb;
            }
        }
    }
    return AR_OK;
}
