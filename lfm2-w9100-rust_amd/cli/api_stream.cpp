// api_stream.cpp -- `api_stream --model|--validate-only MODEL`: the reference's
// JSONL request loop (Amidwestnoob/lfm2-w9100-rust engine/src/bin/api_stream.rs:1-85)
// over the HIP engine, for token-id requests.
//
// One request per stdin line, {"id": str, "tokens": [u32...], "n": 1..1024} (with
// exactly one of "tokens", "text", "chat"; unknown fields rejected), answered by
// JSONL events on stdout with the reference's types and key order: "ready" once
// the model is resident, then per request "accepted", one "delta" per generated
// token and a "result" ("finish_reason" "length" when n tokens were produced,
// else "stop" at the model's EOS id), or a "validation_error".  --validate-only
// checks requests without loading the model ("validated" / "validation_error").
//
// Each request starts a fresh session (conv state cleared) and prefills its
// prompt in chunks of 64 tokens through lfm_forward_token (api_stream.rs:57-63,
// work_bound.rs PREFILL_CHUNK), then feeds each greedy token back one at a time.
// Text is the tokenizer's: "text" and "chat" requests get a validation_error
// (they need the reference's tokenizer and chat template), and the "text" fields
// of "delta" and "result" are null.  Error messages carry the reference's wording
// for its own checks; JSON syntax and type errors are worded by this parser.
#include <unistd.h>

#include <iostream>
#include <string>
#include <vector>

#include "driver.h"
#include "json.h"

using namespace lfmcli;
using lfmjson::Val;

namespace {

constexpr uint32_t kPrefillChunk = 64;

struct Request {
    std::string id;
    bool has_text = false, has_chat = false, has_tokens = false;
    std::vector<uint32_t> tokens;
    uint64_t n = 0;
};

std::string invalid_type(const Val &v, const char *expected)
{
    return std::string("invalid type: ") + lfmjson::kind_name(v) + ", expected " + expected;
}

// serde's derive(Deserialize) with deny_unknown_fields for
// Request { id: String, text: Option<String>, chat: Option<Value>,
//           tokens: Option<Vec<u32>>, n: usize } (api_stream.rs:9-11).
Request decode_request(const std::string &line)
{
    Val v;
    std::string err;
    if (!lfmjson::Parser(line).parse(&v, &err))
        throw Fail(err);
    if (v.kind != Val::Object)
        throw Fail(invalid_type(v, "struct Request"));
    Request r;
    bool seen_id = false, seen_text = false, seen_chat = false, seen_tokens = false, seen_n = false;
    for (const auto &kv : v.obj) {
        const std::string &k = kv.first;
        const Val &x = kv.second;
        bool *seen = k == "id" ? &seen_id
                     : k == "text" ? &seen_text
                     : k == "chat" ? &seen_chat
                     : k == "tokens" ? &seen_tokens
                     : k == "n" ? &seen_n
                                : nullptr;
        if (!seen)
            throw Fail("unknown field `" + k + "`, expected one of `id`, `text`, `chat`, "
                       "`tokens`, `n`");
        if (*seen)
            throw Fail("duplicate field `" + k + "`");
        *seen = true;
        if (k == "id") {
            if (x.kind != Val::Str)
                throw Fail(invalid_type(x, "a string"));
            r.id = x.text;
        } else if (k == "text") {
            if (x.kind != Val::Null && x.kind != Val::Str)
                throw Fail(invalid_type(x, "a string"));
            r.has_text = x.kind == Val::Str;
        } else if (k == "chat") {
            r.has_chat = x.kind != Val::Null;
        } else if (k == "tokens") {
            if (x.kind == Val::Null)
                continue;
            if (x.kind != Val::Arr)
                throw Fail(invalid_type(x, "a sequence"));
            r.has_tokens = true;
            for (const Val &e : x.arr) {
                uint64_t id;
                if (!lfmjson::to_unsigned(e, UINT32_MAX, &id))
                    throw Fail(e.kind == Val::Num && e.integer
                                   ? "invalid value: integer `" + e.text + "`, expected u32"
                                   : invalid_type(e, "u32"));
                r.tokens.push_back((uint32_t)id);
            }
        } else {
            if (!lfmjson::to_unsigned(x, UINT64_MAX, &r.n))
                throw Fail(x.kind == Val::Num && x.integer
                               ? "invalid value: integer `" + x.text + "`, expected usize"
                               : invalid_type(x, "usize"));
        }
    }
    if (!seen_id)
        throw Fail("missing field `id`");
    if (!seen_n)
        throw Fail("missing field `n`");
    return r;
}

// prepare (api_stream.rs:12-27): the same checks in the same order.
Request prepare(const std::string &line, uint64_t bound)
{
    Request r = decode_request(line);
    if (r.id.empty() || r.id.size() > 128)
        throw Fail("invalid id");
    if (r.n < 1 || r.n > 1024)
        throw Fail("max_tokens must be 1..1024");
    if ((int)r.has_text + (int)r.has_chat + (int)r.has_tokens != 1)
        throw Fail("exactly one input required");
    if (!r.has_tokens)
        throw Fail("text and chat requests need the reference's tokenizer and chat template; "
                   "send token ids");
    if (r.tokens.empty() || r.tokens.size() + r.n > 4096)
        throw Fail("empty or context exceeds 4096");
    for (uint32_t id : r.tokens)
        if (id >= bound)
            throw Fail("out-of-range token");
    return r;
}

int run(int argc, char **argv)
{
    const std::string mode = argc == 3 ? argv[1] : "";
    if (mode != "--model" && mode != "--validate-only")
        throw Fail("usage: api_stream --model|--validate-only MODEL");
    const Clock::time_point start = Clock::now();
    Gguf model(argv[2]);
    const uint64_t bound = token_bound(model.g);
    std::string line;
    if (mode == "--validate-only") {
        while (std::getline(std::cin, line)) {
            try {
                const Request r = prepare(line, bound);
                lfmjson::emit(stdout, lfmjson::Obj().s("type", "validated").s("id", r.id)
                                          .list("prompt_tokens", r.tokens));
            } catch (const Fail &e) {
                lfmjson::emit(stdout, lfmjson::Obj().s("type", "validation_error")
                                          .s("message", e.what()));
            }
        }
        return 0;
    }

    // co-resident headroom (api_stream.rs:42-47): free device memory must exceed
    // the weights plus 768 MiB
    uint64_t free_b = 0, total_b = 0;
    check(lfm_device_mem_info(env_device(), &free_b, &total_b));
    const uint64_t used = total_b - free_b, weights = weight_bytes(model.g);
    if (free_b <= weights + (768ull << 20))
        throw Fail("insufficient co-resident VRAM headroom");
    Engine engine;
    load_engine(model.g, LFM_MAX_CTX, &engine);
    const unsigned pid = (unsigned)getpid();
    lfmjson::emit(stdout, lfmjson::Obj().s("type", "ready").u("model_load_count", 1).u("pid", pid)
                              .f("load_ms", ms_since(start)).u("vram_before", used)
                              .u("weight_bytes", weights));
    uint64_t count = 0;
    while (std::getline(std::cin, line)) {
        Request r;
        try {
            r = prepare(line, bound);
        } catch (const Fail &e) {
            lfmjson::emit(stdout, lfmjson::Obj().s("type", "validation_error")
                                      .s("message", e.what())
                                      .u("gpu_dispatches", lfm_dispatch_count(engine.e)));
            continue;
        }
        const std::vector<uint32_t> &prompt = r.tokens;
        lfmjson::emit(stdout, lfmjson::Obj().s("type", "accepted").s("id", r.id)
                                  .list("prompt_tokens", prompt)
                                  .u("gpu_dispatches", lfm_dispatch_count(engine.e)));
        const Clock::time_point t0 = Clock::now();
        check(lfm_reset_session(engine.e));
        uint32_t pos = 0, next = 0;
        float top;
        for (size_t c = 0; c < prompt.size(); c += kPrefillChunk) {
            const uint32_t len = (uint32_t)std::min<size_t>(kPrefillChunk, prompt.size() - c);
            check(lfm_forward_token(engine.e, prompt.data() + c, len, pos, &next, &top));
            pos += len;
        }
        const double prefill_ms = ms_since(t0);
        std::vector<uint32_t> out;
        for (uint64_t i = 0; i < r.n; ++i) {
            const uint32_t token = next;
            if (token == engine.hp.eos)
                break;
            out.push_back(token);
            lfmjson::emit(stdout, lfmjson::Obj().s("type", "delta").s("id", r.id).null("text")
                                      .u("token", token));
            check(lfm_forward_token(engine.e, &token, 1, pos, &next, &top));
            pos += 1;
        }
        ++count;
        lfmjson::emit(stdout, lfmjson::Obj().s("type", "result").s("id", r.id)
                                  .list("prompt_tokens", prompt).list("tokens", out).null("text")
                                  .s("finish_reason", out.size() == r.n ? "length" : "stop")
                                  .u("request_count", count).u("model_load_count", 1)
                                  .u("pid", pid).f("prefill_ms", prefill_ms)
                                  .f("request_ms", ms_since(t0))
                                  .u("gpu_dispatches", lfm_dispatch_count(engine.e)));
    }
    return 0;
}

} // namespace

int main(int argc, char **argv)
{
    try {
        return run(argc, argv);
    } catch (const std::exception &e) {
        fprintf(stderr, "Error: %s\n", e.what());
        return 1;
    }
}
