// lfm2_greedy.cpp -- `lfm2-greedy --model M.gguf --tokens IDS [--n N] [--eos ID]`:
// the reference's greedy CLI (Amidwestnoob/lfm2-w9100-rust engine/src/main.rs:14-280)
// in its --tokens form, over the HIP engine.
//
// Same argument grammar and checks (main.rs:28-113), same generation rule
// (argmax of the prompt's logits, then each argmax fed back, stopping before
// the EOS id, at most --n tokens), the BENCH_TIMING line on stderr
// (main.rs:269-272) and the result object on stdout (main.rs:273-280) with its
// keys in the same order.  Text is the tokenizer's: --text, --chat-json and
// --stream (which need the reference's tokenizer, chat template and stream
// decoder) are rejected, and "decoded_text" is null.  --cpu (the reference's CPU
// diagnostic path) is rejected.  LFM_LOGITS_OUT and LFM_FORWARD_OUT_DIR write
// logits as the reference does (main.rs:155-165, 214-218).
//
// Without LFM_FORWARD_OUT_DIR the tokens after the first come from
// lfm_decode_run, the greedy loop resident on the device; the reference's last
// forward (whose logits nothing reads) is not run.
#include <string>
#include <vector>

#include "driver.h"
#include "json.h"

using namespace lfmcli;

namespace {

enum class Input { None, Tokens, Text, Chat };

struct Args {
    std::string model;
    bool have_model = false;
    Input input = Input::None;
    std::string value;
    uint64_t n = 64;
    uint32_t eos = 124900;
    bool stream = false, cpu = false;
};

// main.rs:28-70
Args parse_args(int argc, char **argv)
{
    Args a;
    for (int i = 1; i < argc; ++i) {
        const std::string arg = argv[i];
        if (arg == "--stream") {
            a.stream = true;
        } else if (arg == "--cpu") {
            a.cpu = true;
        } else if (arg == "--model" || arg == "--tokens" || arg == "--text" ||
                   arg == "--chat-json" || arg == "--n" || arg == "--eos") {
            if (i + 1 >= argc)
                throw Fail(arg + " needs a value");
            const std::string value = argv[++i];
            if (arg == "--model") {
                a.model = value;
                a.have_model = true;
            } else if (arg == "--n") {
                a.n = parse_uint(value, UINT64_MAX);
            } else if (arg == "--eos") {
                a.eos = (uint32_t)parse_uint(value, UINT32_MAX);
            } else {
                if (a.input != Input::None)
                    throw Fail("choose exactly one of --tokens, --text, --chat-json");
                a.input = arg == "--tokens" ? Input::Tokens
                          : arg == "--text" ? Input::Text
                                            : Input::Chat;
                a.value = value;
            }
        } else {
            throw Fail("unknown arg " + arg);
        }
    }
    if (a.input == Input::None)
        throw Fail("need --tokens, --text or --chat-json");
    if (a.cpu && !(a.input == Input::Tokens && !a.stream))
        throw Fail("--cpu is only an explicit --tokens diagnostic; text/chat/stream require the GPU");
    if (!a.have_model)
        throw Fail("need --model");
    return a;
}

// Rust's {:?} of a token string, for the error message.
std::string quoted(const std::string &s)
{
    std::string o = "\"";
    for (char c : s) {
        if (c == '"' || c == '\\')
            o += '\\';
        o += c;
    }
    return o + "\"";
}

// main.rs:71-77: comma-separated ids, whitespace around each ignored, empty
// items skipped.
std::vector<uint32_t> parse_tokens(const std::string &s)
{
    std::vector<uint32_t> ids;
    size_t start = 0;
    for (;;) {
        const size_t end = s.find(',', start);
        std::string item = s.substr(start, end == std::string::npos ? std::string::npos : end - start);
        const size_t a = item.find_first_not_of(" \t\n\r\f\v");
        const size_t b = item.find_last_not_of(" \t\n\r\f\v");
        item = a == std::string::npos ? "" : item.substr(a, b - a + 1);
        if (!item.empty()) {
            try {
                ids.push_back((uint32_t)parse_uint(item, UINT32_MAX));
            } catch (const Fail &) {
                throw Fail("bad token id " + quoted(item));
            }
        }
        if (end == std::string::npos)
            break;
        start = end + 1;
    }
    return ids;
}

// main.rs:114-140: the first index of the largest value; NaN never wins and an
// all-NaN or all -inf vector gives 0.
uint32_t argmax(const std::vector<float> &v)
{
    uint32_t best = 0;
    float value = -INFINITY;
    for (size_t i = 0; i < v.size(); ++i)
        if (v[i] > value) {
            best = (uint32_t)i;
            value = v[i];
        }
    return best;
}

void write_f32(const std::string &path, const std::vector<float> &v)
{
    FILE *f = fopen(path.c_str(), "wb");
    if (!f || fwrite(v.data(), 4, v.size(), f) != v.size() || fclose(f) != 0)
        throw Fail("write " + path + " failed");
}

int run(int argc, char **argv)
{
    const Clock::time_point load_start = Clock::now(), tokenize_start = Clock::now();
    const Args args = parse_args(argc, argv);
    if (args.input != Input::Tokens)
        throw Fail("--text and --chat-json need the reference's tokenizer and chat template; "
                   "this driver takes --tokens");
    if (args.stream)
        throw Fail("--stream needs the reference's stream decoder; this driver prints the "
                   "result object only");
    if (args.cpu)
        throw Fail("--cpu selects the reference's CPU diagnostic path; this driver runs the "
                   "HIP engine");
    Gguf model(args.model);
    const std::vector<uint32_t> prompt = parse_tokens(args.value);
    if (prompt.empty())
        throw Fail("prompt token list must not be empty");
    const uint64_t bound = token_bound(model.g);
    for (uint32_t id : prompt)
        if (id >= bound)
            throw Fail("prompt contains an out-of-range token ID");
    const double tokenize_ms = ms_since(tokenize_start);
    uint64_t ctx;
    if (__builtin_add_overflow((uint64_t)prompt.size(), args.n, &ctx) ||
        __builtin_add_overflow(ctx, (uint64_t)16, &ctx))
        throw Fail("context length overflow");
    if (ctx > LFM_MAX_CTX)
        throw Fail("context " + std::to_string(ctx) + " (prompt + n + 16) exceeds " +
                   std::to_string(LFM_MAX_CTX) + " tokens");

    Engine engine;
    load_engine(model.g, (uint32_t)ctx, &engine);
    if (getenv("LFM_TRACE"))
        fprintf(stderr, "[trace] load complete, device=%s\n", engine.device_name().c_str());
    uint32_t eos = args.eos;
    if (eos == 124900)
        eos = engine.hp.eos;
    const double load_ms = ms_since(load_start);

    const uint32_t P = (uint32_t)prompt.size();
    std::vector<float> logits(engine.hp.vocab);
    const Clock::time_point prompt_start = Clock::now();
    check(lfm_forward_logits(engine.e, prompt.data(), P, 0, logits.data(), logits.size()));
    const double prompt_ms = ms_since(prompt_start);
    const char *keep_dir = getenv("LFM_FORWARD_OUT_DIR");
    if (keep_dir)
        write_f32(std::string(keep_dir) + "/forward-0.logits.bin", logits);
    if (const char *path = getenv("LFM_LOGITS_OUT"))
        write_f32(path, logits);

    std::vector<uint32_t> out;
    const Clock::time_point gen_start = Clock::now();
    if (keep_dir) {
        // every step's logits on the host, as main.rs:192-219
        for (uint64_t step = 0; step < args.n; ++step) {
            const uint32_t token = argmax(logits);
            if (token == eos)
                break;
            out.push_back(token);
            check(lfm_forward_logits(engine.e, &token, 1, P + (uint32_t)step, logits.data(),
                                     logits.size()));
            write_f32(std::string(keep_dir) + "/forward-" + std::to_string(step + 1) +
                          ".logits.bin",
                      logits);
        }
    } else if (args.n > 0) {
        const uint32_t first = argmax(logits);
        if (first != eos) {
            out.push_back(first);
            if (args.n > 1) {
                std::vector<uint32_t> more(args.n - 1);
                uint32_t got = 0;
                check(lfm_decode_run(engine.e, first, P, (uint32_t)(args.n - 1), eos, more.data(),
                                     &got));
                out.insert(out.end(), more.begin(), more.begin() + got);
            }
        }
    }
    const double gen_ms = ms_since(gen_start);

    lfmjson::Obj timing;
    timing.f("load_ms", load_ms).f("tokenize_ms", tokenize_ms).f("warmup_ms", 0.0)
        .f("prompt_ms", prompt_ms).f("gen_ms", gen_ms).u("n_prompt_tokens", prompt.size())
        .u("n_gen_tokens", out.size());
    fprintf(stderr, "BENCH_TIMING %s\n", timing.text().c_str());
    fflush(stderr);
    lfmjson::Obj result;
    result.list("prompt_tokens", prompt).list("tokens", out).null("decoded_text")
        .b("greedy", true).s("device", engine.device_name())
        .u("gpu_dispatch_count", lfm_dispatch_count(engine.e)).u("eos", eos)
        .u("n_vocab", engine.hp.vocab);
    lfmjson::emit(stdout, result);
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
