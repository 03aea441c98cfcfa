// ar_train.cpp -- the training driver: a C++ restatement of train.mojo's
// main (train.mojo:128-339) over the library's C ABI (include/ar_ops.h,
// include/ar_data.h).
//
// Same loop and arithmetic as the reference: zero_grads -> forward ->
// backward, next batch, progress = training_time / budget, AdamW + Muon
// (ar_gpt_optimizer_step applies train.mojo:25-33 and 246-281), NaN /
// explosion fast-fail, the first 11 steps excluded from training_time, the
// same per-step log line and final summary block, then validation bits per
// byte (train.mojo:67-123).  Differences:
//   * data: pre-tokenized token shards (ar_data.h) instead of parquet +
//     the BPE tokenizer, which are not part of this build;
//   * the next batch is packed on the host while the GPU runs forward and
//     backward, into the other of two device token buffers;
//   * --graph replays the whole step from a HIP graph (ar_gpt_train_step_graph,
//     bit-identical to the eager step).
//
// Usage: ar_train [--data DIR] [--tokenizer DIR] [--vocab V] [--depth D]
//                 [--batch B] [--seq T] [--fp32] [--graph] [--fake-dt SEC]
//                 [--nan-at STEP]
//   TRAIN_TIME_BUDGET=<seconds> overrides the 300 s budget (train.mojo:211-221).
//   --fake-dt replaces each step's measured time in the schedule (tests).
//   --nan-at writes a NaN into lm_head before step STEP (tests of the NaN
//     fast fail, train.mojo:284-287; the kernels run normally on NaN data).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <chrono>
#include <string>
#include <vector>

#include "ar_data.h"
#include "ar_ops.h"

namespace {

constexpr int kTimeBudget = 300;     // config.mojo:61
constexpr int kDepth = 8;            // config.mojo:62
constexpr int kMaxSeqLen = 2048;     // config.mojo:60
constexpr int kVocab = 8192;         // prepare.py:45
constexpr int kWarmupSteps = 10;     // train.mojo:291-293: steps 0..10 untimed

double now_s() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// Float64 printed as its shortest round-trip decimal, always with a '.' or
// exponent ("1.0", not "1"), the form the reference's log shows.
std::string f64(double x) {
    if (isnan(x)) return "nan";
    if (isinf(x)) return x > 0 ? "inf" : "-inf";
    char buf[64];
    for (int p = 15; p <= 17; ++p) {
        snprintf(buf, sizeof buf, "%.*g", p, x);
        if (strtod(buf, nullptr) == x) break;
    }
    std::string s = buf;
    if (s.find_first_of(".en") == std::string::npos) s += ".0";
    return s;
}

[[noreturn]] void die(const char* what) {
    fprintf(stderr, "ERROR: %s: %s\n", what, ar_last_error());
    exit(1);
}
#define CHECK(call, what)                 \
    do {                                  \
        if ((call) != AR_OK) die(what);   \
    } while (0)
#define HIPCHECK(call, what)                                                   \
    do {                                                                       \
        hipError_t e_ = (call);                                                \
        if (e_ != hipSuccess) {                                                \
            fprintf(stderr, "ERROR: %s: %s\n", what, hipGetErrorString(e_));   \
            exit(1);                                                           \
        }                                                                      \
    } while (0)

// train.mojo:25-33
double lr_multiplier(double progress) {
    const double warmup = 0.0, warmdown = 0.5, final_frac = 0.0;  // config.mojo:81-83
    if (progress < warmup) return warmup > 0 ? progress / warmup : 1.0;
    if (progress < 1.0 - warmdown) return 1.0;
    const double cd = (1.0 - progress) / warmdown;
    return cd + (1.0 - cd) * final_frac;
}

struct Args {
    std::string data, tok;
    int64_t vocab = kVocab, depth = kDepth, B = 4, T = 512;  // train.mojo:152-153
    bool fp32 = false, graph = false;
    double fake_dt = -1.0;
    int64_t nan_at = -1;  // --nan-at STEP: lm_head[0] := NaN before that step (tests the fast fail)
};

Args parse(int argc, char** argv) {
    Args a;
    const char* home = getenv("HOME");
    const std::string cache = std::string(home ? home : ".") + "/.cache/autoresearch";
    a.data = cache + "/data";
    a.tok = cache + "/tokenizer";
    for (int i = 1; i < argc; ++i) {
        const std::string k = argv[i];
        auto val = [&]() -> const char* {
            if (i + 1 >= argc) {
                fprintf(stderr, "ERROR: %s needs a value\n", k.c_str());
                exit(2);
            }
            return argv[++i];
        };
        if (k == "--data") a.data = val();
        else if (k == "--tokenizer") a.tok = val();
        else if (k == "--vocab") a.vocab = atoll(val());
        else if (k == "--depth") a.depth = atoll(val());
        else if (k == "--batch") a.B = atoll(val());
        else if (k == "--seq") a.T = atoll(val());
        else if (k == "--fp32") a.fp32 = true;
        else if (k == "--graph") a.graph = true;
        else if (k == "--fake-dt") a.fake_dt = atof(val());
        else if (k == "--nan-at") a.nan_at = atoll(val());
        else {
            fprintf(stderr, "usage: ar_train [--data DIR] [--tokenizer DIR] [--vocab V] [--depth D] [--batch B] "
                            "[--seq T] [--fp32] [--graph] [--fake-dt SEC] [--nan-at STEP]\n");
            exit(2);
        }
    }
    return a;
}

// config.mojo:24-44 (GPTConfig.default)
ar_gpt_config default_config(int64_t vocab, int64_t depth) {
    const int64_t head_dim = 128;
    const int64_t model_dim = ((depth * 64 + head_dim - 1) / head_dim) * head_dim;
    const int64_t nh = model_dim / head_dim;
    return ar_gpt_config{kMaxSeqLen, vocab, depth, nh, nh, model_dim, model_dim / nh, nh * (model_dim / nh)};
}

}  // namespace

int main(int argc, char** argv) {
    const Args a = parse(argc, argv);
    printf("=== Autoresearch Training (MI355X) ===\n\n");
    const double t_start = now_s();

    const ar_gpt_config cfg = default_config(a.vocab, a.depth);
    const int64_t B = a.B, T = a.T, BT = B * T, V = cfg.vocab_size;
    printf("Model: L= %lld  H= %lld  C= %lld  V= %lld\n", (long long)cfg.n_layer, (long long)cfg.n_head,
           (long long)cfg.n_embd, (long long)V);
    printf("Batch: B= %lld  T= %lld  tokens/step= %lld\n", (long long)B, (long long)T, (long long)BT);
    fflush(stdout);

    std::vector<int32_t> token_bytes((size_t)V);
    CHECK(ar_token_bytes_load((a.tok + "/token_bytes.bin").c_str(), token_bytes.data(), V), "token_bytes");

    hipStream_t st;
    HIPCHECK(hipStreamCreate(&st), "stream");
    ar_stream_t ast = reinterpret_cast<ar_stream_t>(st);
    // RoPE positions: the flat token index while B*T fits the reference's
    // MAX_SEQ_LEN-row table (as train.mojo's B4 T512 step does), else t mod T.
    const int64_t rope_period = BT <= kMaxSeqLen ? 0 : T;
    ar_gpt* m = nullptr;
    CHECK(ar_gpt_create(&m, &cfg, B, T, a.fp32 ? AR_PREC_FP32 : AR_PREC_BF16, rope_period, ast), "gpt_create");
    CHECK(ar_gpt_init_weights(m, 42), "init_weights");  // model.mojo:347

    ar_loader* train = nullptr;
    CHECK(ar_loader_create(&train, a.data.c_str(), "train", B, T, 1000), "train loader");
    int64_t *h_in, *h_tg;  // pinned host batch
    HIPCHECK(hipHostMalloc((void**)&h_in, BT * sizeof(int64_t), hipHostMallocDefault), "pinned");
    HIPCHECK(hipHostMalloc((void**)&h_tg, BT * sizeof(int64_t), hipHostMallocDefault), "pinned");
    int64_t* d_tok[2][2];  // [buffer][inputs, targets]
    for (auto& b : d_tok)
        for (auto& p : b) HIPCHECK(hipMalloc((void**)&p, BT * sizeof(int64_t)), "token buffers");
    int cur = 0;
    int64_t epoch = 1;
    auto upload = [&](int buf) {
        HIPCHECK(hipMemcpyAsync(d_tok[buf][0], h_in, BT * sizeof(int64_t), hipMemcpyHostToDevice, st), "upload");
        HIPCHECK(hipMemcpyAsync(d_tok[buf][1], h_tg, BT * sizeof(int64_t), hipMemcpyHostToDevice, st), "upload");
        HIPCHECK(hipStreamSynchronize(st), "upload");
    };
    CHECK(ar_loader_next(train, h_in, h_tg, &epoch), "load batch");
    upload(cur);

    int time_budget = kTimeBudget;
    if (const char* s = getenv("TRAIN_TIME_BUDGET"))
        if (*s) time_budget = atoi(s);
    printf("Time budget: %d s\n\n", time_budget);
    fflush(stdout);

    const double t_train_start = now_s();
    double training_time = 0.0, smooth_loss = 0.0;
    int64_t step = 0;
    for (;;) {
        const double t0 = now_s();
        // progress depends on the time of the finished steps only, so it is
        // known before this step's forward (train.mojo:247-250)
        double progress = training_time / (double)time_budget;
        if (progress > 1.0) progress = 1.0;
        const double lrm = lr_multiplier(progress);
        int64_t next_epoch = epoch;
        float loss32 = 0.f;
        if (step == a.nan_at) {
            // fault injection from the host: one lm_head weight becomes NaN, so
            // every logit row, and the step's loss, is NaN
            int64_t off = -1;
            for (int64_t i = 0; i < ar_gpt_num_tensors(m); ++i) {
                int64_t o = 0;
                const char* nm = nullptr;
                ar_gpt_tensor_info(m, i, &o, &nm);
                if (nm && std::string(nm) == "lm_head") off = o;
            }
            const float qnan = NAN;
            HIPCHECK(off >= 0 ? hipSuccess : hipErrorInvalidValue, "lm_head offset");
            HIPCHECK(hipMemcpyAsync(ar_gpt_params(m) + off, &qnan, sizeof(float), hipMemcpyHostToDevice, st), "nan");
            HIPCHECK(hipStreamSynchronize(st), "nan");
        }
        if (a.graph) {
            // one graph replay (zero_grads -> forward -> backward -> AdamW + Muon)
            // on the fixed token buffers; the next batch is packed meanwhile
            CHECK(ar_gpt_train_step_graph(m, d_tok[0][0], d_tok[0][1], progress, nullptr), "graph step");
            CHECK(ar_loader_next(train, h_in, h_tg, &next_epoch), "load batch");
            HIPCHECK(hipMemcpyAsync(&loss32, ar_gpt_mean_loss(m), sizeof(float), hipMemcpyDeviceToHost, st), "loss");
            HIPCHECK(hipStreamSynchronize(st), "step");
            upload(0);
        } else {
            CHECK(ar_gpt_zero_grads(m), "zero_grads");
            CHECK(ar_gpt_forward(m, d_tok[cur][0], d_tok[cur][1], nullptr), "forward");
            CHECK(ar_gpt_backward(m, d_tok[cur][0], d_tok[cur][1], 1.0f), "backward");
            // the next batch is packed while the GPU works
            CHECK(ar_loader_next(train, h_in, h_tg, &next_epoch), "load batch");
            HIPCHECK(hipMemcpyAsync(&loss32, ar_gpt_mean_loss(m), sizeof(float), hipMemcpyDeviceToHost, st), "loss");
            HIPCHECK(hipStreamSynchronize(st), "step");
            upload(cur ^ 1);
            CHECK(ar_gpt_optimizer_step(m, progress), "optimizer");
            HIPCHECK(hipStreamSynchronize(st), "optimizer");
            cur ^= 1;
        }
        const double loss = loss32;
        epoch = next_epoch;

        if (isnan(loss) || loss > 100.0) {  // train.mojo:285-287
            printf("FAIL: loss = %s\n", f64(loss).c_str());
            return 0;
        }
        const double t1 = now_s();
        const double dt = a.fake_dt >= 0 ? a.fake_dt : t1 - t0;
        if (step > kWarmupSteps) training_time += dt;

        smooth_loss = 0.9 * smooth_loss + 0.1 * loss;
        const double debiased = smooth_loss / (1.0 - pow(0.9, (double)(step + 1)));
        double remaining = (double)time_budget - training_time;
        if (remaining < 0) remaining = 0;
        printf("step %lld  | %d %% |  loss: %s  | lrm: %s  | dt: %d ms  | epoch: %lld  | rem: %d s\n",
               (long long)step, (int)(100.0 * progress), f64(debiased).c_str(), f64(lrm).c_str(), (int)(dt * 1000),
               (long long)epoch, (int)remaining);
        fflush(stdout);
        ++step;
        if (step > kWarmupSteps && training_time >= (double)time_budget) break;
    }

    // train.mojo:67-123 (evaluate_bpb)
    printf("\nEvaluating validation BPB...\n");
    fflush(stdout);
    ar_loader* val = nullptr;
    CHECK(ar_loader_create(&val, a.data.c_str(), "val", B, T, 1000), "val loader");
    int64_t eval_steps = 40 * 524288 / BT;
    if (eval_steps > 100) eval_steps = 100;
    std::vector<float> tok_loss((size_t)BT);
    double nats = 0.0, nbytes = 0.0;
    for (int64_t i = 0; i < eval_steps; ++i) {
        int64_t e;
        CHECK(ar_loader_next(val, h_in, h_tg, &e), "val batch");
        upload(0);
        CHECK(ar_gpt_forward(m, d_tok[0][0], d_tok[0][1], nullptr), "eval forward");
        HIPCHECK(hipMemcpyAsync(tok_loss.data(), ar_gpt_token_loss(m), BT * sizeof(float), hipMemcpyDeviceToHost, st),
                 "eval loss");
        HIPCHECK(hipStreamSynchronize(st), "eval");
        CHECK(ar_bpb_accumulate(tok_loss.data(), h_tg, token_bytes.data(), BT, V, &nats, &nbytes), "bpb");
    }
    const double val_bpb = nbytes > 0 ? nats / (0.6931471805599453 * nbytes) : 0.0;

    const double t_end = now_s();
    printf("\n---\n");
    printf("val_bpb:          %s\n", f64(val_bpb).c_str());
    printf("training_seconds: %s\n", f64(training_time).c_str());
    printf("total_seconds:    %s\n", f64(t_end - t_start).c_str());
    printf("startup_seconds:  %s\n", f64(t_train_start - t_start).c_str());
    printf("total_tokens_M:   %s\n", f64((double)(step * BT) / 1e6).c_str());
    printf("num_steps:        %lld\n", (long long)step);
    printf("depth:            %lld\n", (long long)a.depth);
    fflush(stdout);

    ar_loader_destroy(val);
    ar_loader_destroy(train);
    ar_gpt_destroy(m);
    for (auto& b : d_tok)
        for (auto& p : b) hipFree(p);
    hipHostFree(h_in);
    hipHostFree(h_tg);
    hipStreamDestroy(st);
    return 0;
}
