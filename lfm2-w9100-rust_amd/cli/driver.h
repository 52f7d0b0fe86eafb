// driver.h -- model loading and errors shared by the command-line drivers.
//
// Environment (read by both drivers):
//   LFM_ANY_GEOMETRY=1  accept any geometry the engine supports; by default the
//                       model must have the LFM2.5-8B-A1B geometry, as the
//                       reference's load_hyperparams requires (engine/src/lfm.rs:117-130)
//   LFM_DEVICE=N        HIP device index (default 0)
#pragma once

#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/lfm_hip.h"

namespace lfmcli {

// Any failure: main prints "Error: <message>" on stderr and exits with status 1,
// as a Rust main returning Err does.
struct Fail : std::runtime_error {
    explicit Fail(const std::string &m) : std::runtime_error(m) {}
};

inline void check(int rc)
{
    if (rc != LFM_OK)
        throw Fail(lfm_last_error());
}

inline bool env_flag(const char *name)
{
    const char *v = getenv(name);
    return v && *v && strcmp(v, "0") != 0;
}

inline int env_device()
{
    const char *v = getenv("LFM_DEVICE");
    return v && *v ? atoi(v) : 0;
}

using Clock = std::chrono::steady_clock;
inline double ms_since(Clock::time_point t0)
{
    return std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
}

// Rust's u64 FromStr: an optional '+', then decimal digits only, within `max`.
// The messages are those of Rust's ParseIntError.
inline uint64_t parse_uint(const std::string &s, uint64_t max)
{
    size_t i = 0;
    if (s.empty())
        throw Fail("cannot parse integer from empty string");
    if (s[0] == '+')
        i = 1;
    if (i == s.size())
        throw Fail("invalid digit found in string");
    uint64_t x = 0;
    for (; i < s.size(); ++i) {
        if (s[i] < '0' || s[i] > '9')
            throw Fail("invalid digit found in string");
        const uint64_t d = (uint64_t)(s[i] - '0');
        if (x > (max - d) / 10)
            throw Fail("number too large to fit in target type");
        x = x * 10 + d;
    }
    return x;
}

// Owns an open GGUF file.
struct Gguf {
    lfm_gguf *g = nullptr;
    explicit Gguf(const std::string &path) { check(lfm_gguf_open(path.c_str(), &g)); }
    ~Gguf() { lfm_gguf_close(g); }
    Gguf(const Gguf &) = delete;
    Gguf &operator=(const Gguf &) = delete;
};

// Owns an engine.
struct Engine {
    lfm_engine *e = nullptr;
    lfm_hparams hp{};
    Engine() = default;
    ~Engine() { lfm_engine_destroy(e); }
    Engine(const Engine &) = delete;
    Engine &operator=(const Engine &) = delete;

    std::string device_name() const
    {
        char buf[256];
        check(lfm_device_name(e, buf, sizeof(buf)));
        return buf;
    }
};

// Tokenizer::vocab_size (tokenizer/src/vocab.rs:676-678) is the number of
// entries of tokenizer.ggml.tokens; a file without tokenizer tables (the seeded
// synthetic models) bounds token ids by lfm2moe.vocab_size.
inline uint64_t token_bound(const lfm_gguf *g)
{
    lfm_gguf_value v;
    if (lfm_gguf_meta_get(g, "tokenizer.ggml.tokens", &v) == LFM_OK && v.type == LFM_GGUF_TYPE_ARRAY)
        return v.len;
    uint32_t vocab;
    check(lfm_gguf_meta_u32(g, "lfm2moe.vocab_size", &vocab));
    return vocab;
}

// Sum of every tensor's bytes (the weight_bytes of bin/api_stream.rs:46).
inline uint64_t weight_bytes(const lfm_gguf *g)
{
    uint64_t n = 0, total = 0;
    check(lfm_gguf_header(g, nullptr, nullptr, nullptr, nullptr, &n));
    for (uint64_t i = 0; i < n; ++i) {
        lfm_gguf_tensor t;
        check(lfm_gguf_tensor_info(g, i, &t));
        total += t.nbytes;
    }
    return total;
}

// GpuEngine::load + set_ctx (engine/src/gpu_lfm.rs:51-120).
inline void load_engine(const lfm_gguf *g, uint32_t ctx, Engine *out)
{
    check(lfm_gguf_hparams(g, env_flag("LFM_ANY_GEOMETRY") ? 0 : 1, &out->hp));
    if (out->hp.n_expert < 4 || out->hp.n_expert > 64)
        throw Fail("resident routing supports 4..=64 experts");
    check(lfm_engine_create(&out->hp, env_device(), &out->e));
    check(lfm_engine_set_ctx(out->e, ctx));
    check(lfm_engine_load_gguf(out->e, g));
    check(lfm_engine_finalize(out->e));
}

} // namespace lfmcli
