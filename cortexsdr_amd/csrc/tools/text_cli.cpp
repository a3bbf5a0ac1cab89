// text_cli.cpp — one-shot generation from a .sdr archive through the device path.
//
// The role of the reference's cortexsdr_text_cli (src/cortexsdr_cli.cpp:1460-1713): same
// flags for the one-shot path (-p/--prompt, -m/--max-length, --profile FILE, -h, -v, the model
// path last) and the same profile JSON (duration_ms, tokens, tokens_per_sec, engine_stats),
// so the reference's bench suite runner can drive it. The prompt is whitespace-separated
// token ids (no tokenizer on this path) and the output is the generated ids.
//
//   cortexsdr_text_cli -p "1 2 3" -m 64 --profile out.json model.sdr
//
// --lazy-hsdr packed|cli chooses tokens as the reference CLI's native path does with an HSDR
// token embedding (select_next_token_from_lazy_hsdr, cortexsdr_cli.cpp:687-732): the codes
// read as written (packed) or with the CLI's own reading (cli, index = v >> 1, sign = v & 1).
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "../../../include/cortex_sdk_gpu.h"

namespace {

void usage(const char* argv0) {
    std::printf(
        "usage: %s [-p|--prompt \"ids\"] [-m|--max-length N] [--profile FILE]\n"
        "          [--lazy-hsdr packed|cli] model.sdr\n"
        "  -p, --prompt      whitespace-separated token ids\n"
        "  -m, --max-length  tokens to generate (default 64)\n"
        "      --profile     write {duration_ms, tokens, tokens_per_sec, engine_stats} JSON\n"
        "      --lazy-hsdr   choose tokens by lazy HSDR scoring of the token embedding\n"
        "                    (codes read as written, or as the reference CLI reads them)\n"
        "  -v, --version     print the SDK version\n",
        argv0);
}

int report(const CortexError& e, const char* what) {
    std::fprintf(stderr, "Error: %s: %s (code %d)\n", what, e.message ? e.message : "", e.code);
    return 1;
}

}  // namespace

int main(int argc, char** argv) {
    std::string prompt, profile, model;
    int max_length = 64;
    int lazy = 0;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if (a == "-h" || a == "--help") {
            usage(argv[0]);
            return 0;
        } else if (a == "-v" || a == "--version") {
            std::printf("cortexsdr_text_cli %s\n", cortex_sdk_version());
            return 0;
        } else if ((a == "-p" || a == "--prompt") && i + 1 < argc) {
            prompt = argv[++i];
        } else if ((a == "-m" || a == "--max-length") && i + 1 < argc) {
            max_length = std::atoi(argv[++i]);
        } else if (a == "--profile" && i + 1 < argc) {
            profile = argv[++i];
        } else if (a == "--lazy-hsdr" && i + 1 < argc) {
            const std::string m = argv[++i];
            lazy = m == "packed" ? 1 : (m == "cli" ? 2 : -1);
            if (lazy < 0) {
                std::fprintf(stderr, "--lazy-hsdr takes packed or cli\n");
                return 2;
            }
        } else if (!a.empty() && a[0] != '-') {
            model = a;
        } else {
            std::fprintf(stderr, "unknown or incomplete option: %s\n", a.c_str());
            usage(argv[0]);
            return 2;
        }
    }
    if (model.empty() || prompt.empty()) {
        usage(argv[0]);
        return 2;
    }
    CortexInferenceEngineHandle h = nullptr;
    CortexError e = cortex_inference_engine_create(model.c_str(), &h);
    if (e.code) return report(e, "create");
    if (lazy) {
        e = cortex_inference_engine_set_lazy_hsdr_selection(h, lazy);
        if (e.code) {
            report(e, "lazy-hsdr");
            cortex_inference_engine_free(h);
            return 1;
        }
    }
    std::printf("Generating response for: %s\n", prompt.c_str());
    const auto t0 = std::chrono::high_resolution_clock::now();
    char* text = nullptr;
    e = cortex_inference_engine_generate_text(h, prompt.c_str(), max_length, &text);
    const auto t1 = std::chrono::high_resolution_clock::now();
    if (e.code) {
        report(e, "generate");
        cortex_inference_engine_free(h);
        return 1;
    }
    const double ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    size_t tokens = 0;
    for (const char* p = text; *p;) {
        while (*p == ' ') ++p;
        if (!*p) break;
        ++tokens;
        while (*p && *p != ' ') ++p;
    }
    const double tps = ms > 0 ? tokens / (ms / 1000.0) : 0.0;
    std::printf("Generated in %.0fms | tokens: %zu | tokens/sec: %.2f\n", ms, tokens, tps);
    std::printf("Response: %s\n", text);
    char* stats = nullptr;
    cortex_inference_engine_get_last_run_stats_json(h, &stats);
    if (!profile.empty()) {
        FILE* f = std::fopen(profile.c_str(), "w");
        if (!f) {
            std::fprintf(stderr, "Error: Could not open profile path: %s\n", profile.c_str());
        } else {
            std::fprintf(f,
                         "{\n  \"duration_ms\": %.0f,\n  \"tokens\": %zu,\n"
                         "  \"tokens_per_sec\": %.2f,\n  \"engine_stats\": %s\n}\n",
                         ms, tokens, tps, stats ? stats : "null");
            std::fclose(f);
            std::printf("Wrote profile to %s\n", profile.c_str());
        }
    }
    cortex_free_string(stats);
    cortex_free_string(text);
    e = cortex_inference_engine_free(h);
    return e.code ? report(e, "free") : 0;
}
