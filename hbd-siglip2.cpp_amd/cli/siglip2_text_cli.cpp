// siglip2-text-cli -- the text encoder from the command line, over the
// drop-in class (include/siglip2_text.h) on libs2x.
//
// The flags, exit codes and messages are those of the reference's
// src/siglip2_text_cli.cpp (its command-line contract):
//   --model GGUF (with t.* tensors), and exactly one input pair:
//     --token-ids FILE --attention-mask FILE: int32 buffers of one length
//         (1 = valid, 0 = pad), as the reference's tokenizer step writes;
//     --tokenizer FILE --text STRING: needs the SentencePiece tokenizer,
//         which this build does not have, so it fails with a message;
//   --out FILE (raw fp32), else a summary on stdout.
// Exit codes: 0 ok, 1 load / read / encode failure, 2 bad arguments.
#include "cli_common.h"
#include "siglip2_text.h"

#include <cstdio>
#include <string>
#include <vector>

namespace {

using namespace s2xcli;

struct Request {
    std::string model, tokenizer, text, ids_file, mask_file, out_file;
    bool from_text() const { return !tokenizer.empty() && !text.empty(); }
    bool from_ids() const { return !ids_file.empty() && !mask_file.empty(); }
};

std::vector<Option> options(Request &r) {
    const struct {
        const char *name, *alias, *meta, *help;
        std::string *dst;
    } rows[] = {
        {"--model", "-m", "<gguf>", "SigLIP2 GGUF with t.* tensors", &r.model},
        {"--token-ids", nullptr, "<file>", "pre-tokenized int32 ids", &r.ids_file},
        {"--attention-mask", nullptr, "<file>", "int32 mask of the same length (1 valid, 0 pad)", &r.mask_file},
        {"--tokenizer", nullptr, "<spm.model>", "SentencePiece model (not in this build)", &r.tokenizer},
        {"--text", nullptr, "<prompt>", "text to tokenize with --tokenizer", &r.text},
        {"--out", nullptr, "<file>", "raw fp32 embedding (default: summary on stdout)", &r.out_file},
    };
    std::vector<Option> t;
    for (const auto &row : rows) {
        Option o{row.name, row.alias, row.meta, row.help};
        o.text = row.dst;
        t.push_back(o);
    }
    return t;
}

void usage(const std::vector<Option> &table, const char *prog) {
    const std::string p(prog);
    print_usage(stderr, "siglip2-text-cli (text encoder, libs2x on gfx950)",
                {p + " --model <gguf> --token-ids tok.bin --attention-mask mask.bin [--out file]",
                 p + " --model <gguf> --tokenizer <spm.model> --text \"prompt\" [--out file]"},
                table);
}

// ids and mask, read and checked against each other
int load_tokens(const Request &r, std::vector<int32_t> &ids, std::vector<int32_t> &mask) {
    std::vector<uint8_t> ib, mb;
    std::string err;
    if (!slurp(r.ids_file, ib, err) || !slurp(r.mask_file, mb, err)) {
        std::fprintf(stderr, "%s\n", err.c_str());
        return EXIT_FAIL;
    }
    if (ib.empty() || ib.size() != mb.size() || ib.size() % sizeof(int32_t) != 0) {
        std::fprintf(stderr, "tok/mask size mismatch or invalid (tok=%zu mask=%zu)\n", ib.size(), mb.size());
        return EXIT_FAIL;
    }
    ids = as_values<int32_t>(ib);
    mask = as_values<int32_t>(mb);
    return 0;
}

int run(const Request &r) {
    siglip2::TextEncoder enc;
    if (!enc.load(r.model)) {
        std::fprintf(stderr, "load failed: %s\n", enc.last_error().c_str());
        return EXIT_FAIL;
    }
    if (r.from_text()) {
        std::fprintf(stderr, "tokenizer load failed: no SentencePiece tokenizer in this build; tokenize "
                             "elsewhere and pass --token-ids / --attention-mask\n");
        return EXIT_FAIL;
    }
    std::vector<int32_t> ids, mask;
    if (const int rc = load_tokens(r, ids, mask)) return rc;
    std::vector<float> emb;
    if (!enc.encode(ids.data(), (int)ids.size(), mask.data(), emb)) {
        std::fprintf(stderr, "encode failed: %s\n", enc.last_error().c_str());
        return EXIT_FAIL;
    }
    if (r.out_file.empty()) {
        print_summary(stdout, "text embedding", emb);
        return EXIT_OK;
    }
    std::string err;
    if (!spill(r.out_file, emb.data(), emb.size() * sizeof(float), err)) {
        std::fprintf(stderr, "%s\n", err.c_str());
        return EXIT_FAIL;
    }
    std::fprintf(stderr, "wrote text embedding (%zu floats) to %s\n", emb.size(), r.out_file.c_str());
    return EXIT_OK;
}

}  // namespace

int main(int argc, char **argv) {
    Request req;
    const std::vector<Option> table = options(req);
    std::string err;
    const Parsed parsed = parse(argc, argv, table, err);
    if (parsed == Parsed::help || parsed == Parsed::bad || req.model.empty()) {
        if (parsed == Parsed::bad) std::fprintf(stderr, "%s\n", err.c_str());
        usage(table, argv[0]);
        return parsed == Parsed::help ? EXIT_OK : EXIT_USAGE;
    }
    if (req.from_text() == req.from_ids()) {
        std::fprintf(stderr, "Provide exactly one of (--tokenizer + --text) or (--token-ids + --attention-mask)\n");
        return EXIT_USAGE;
    }
    return run(req);
}
