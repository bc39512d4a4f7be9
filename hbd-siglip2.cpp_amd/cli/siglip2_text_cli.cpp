// siglip2-text-cli -- the text encoder from the command line, over the
// drop-in class (include/siglip2_text.h) on libs2x.
//
// Same arguments, raw-file contract and exit codes as the reference's
// src/siglip2_text_cli.cpp:16-135:
//   --model GGUF (with t.* tensors), and
//   --token-ids FILE --attention-mask FILE: int32 buffers of one length
//       (1 = valid, 0 = pad), as written by the reference's tokenizer step;
//   --tokenizer + --text: needs the SentencePiece tokenizer, not built
//       here, so it fails with a message;
//   --out FILE (raw fp32), else the first 8 values as text on stdout.
// Exit codes: 0 ok, 1 load / read / encode failure, 2 bad arguments.
#include "siglip2_text.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

namespace {

void usage(const char *argv0) {
    fprintf(stderr,
            "siglip2-text-cli (text encoder, libs2x on gfx950)\n"
            "\n"
            "Usage:\n"
            "  %s --model <gguf> --token-ids tok.bin --attention-mask mask.bin  [--out file]\n"
            "  %s --model <gguf> --tokenizer <spm.model> --text \"prompt\" [--out file]\n"
            "\n"
            "  --model           SigLIP2 GGUF (must have t.* tensors)\n"
            "  --token-ids       pre-tokenized int32 buffer\n"
            "  --attention-mask  same length (1=valid, 0=pad); required with --token-ids\n"
            "  --tokenizer       sentencepiece tokenizer.model: not built here\n"
            "  --text            free-form text input (tokenize via --tokenizer)\n"
            "  --out             write fp32 embedding to this file (default: stdout text)\n",
            argv0, argv0);
}

bool read_bytes(const std::string &path, std::vector<uint8_t> &out, std::string &err) {
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) {
        err = "could not open: " + path;
        return false;
    }
    const std::streamsize n = f.tellg();
    f.seekg(0);
    out.resize((size_t)n);
    f.read(reinterpret_cast<char *>(out.data()), n);
    if (!f.good()) err = "could not read: " + path;
    return f.good();
}

bool write_bytes(const std::string &path, const void *data, size_t bytes, std::string &err) {
    std::ofstream f(path, std::ios::binary);
    if (!f) {
        err = "could not write: " + path;
        return false;
    }
    f.write(reinterpret_cast<const char *>(data), (std::streamsize)bytes);
    if (!f.good()) err = "could not write: " + path;
    return f.good();
}

}  // namespace

int main(int argc, char **argv) {
    std::string model_path, tokenizer_path, text_input, tok_path, mask_path, out_path;
    for (int i = 1; i < argc; ++i) {
        const bool more = i + 1 < argc;
        if ((!strcmp(argv[i], "--model") || !strcmp(argv[i], "-m")) && more)
            model_path = argv[++i];
        else if (!strcmp(argv[i], "--tokenizer") && more)
            tokenizer_path = argv[++i];
        else if (!strcmp(argv[i], "--text") && more)
            text_input = argv[++i];
        else if (!strcmp(argv[i], "--token-ids") && more)
            tok_path = argv[++i];
        else if (!strcmp(argv[i], "--attention-mask") && more)
            mask_path = argv[++i];
        else if (!strcmp(argv[i], "--out") && more)
            out_path = argv[++i];
        else if (!strcmp(argv[i], "--help") || !strcmp(argv[i], "-h")) {
            usage(argv[0]);
            return 0;
        } else {
            fprintf(stderr, "Unknown arg: %s\n", argv[i]);
            usage(argv[0]);
            return 2;
        }
    }
    if (model_path.empty()) {
        usage(argv[0]);
        return 2;
    }
    const bool use_text = !tokenizer_path.empty() && !text_input.empty();
    const bool use_bin = !tok_path.empty() && !mask_path.empty();
    if (use_text == use_bin) {
        fprintf(stderr,
                "Provide exactly one of (--tokenizer + --text) or (--token-ids + --attention-mask)\n");
        return 2;
    }
    siglip2::TextEncoder enc;
    if (!enc.load(model_path)) {
        fprintf(stderr, "load failed: %s\n", enc.last_error().c_str());
        return 1;
    }
    if (use_text) {
        fprintf(stderr,
                "tokenizer load failed: no SentencePiece tokenizer in this build; tokenize "
                "elsewhere and pass --token-ids / --attention-mask\n");
        return 1;
    }
    std::string err;
    std::vector<uint8_t> tok_raw, mask_raw;
    if (!read_bytes(tok_path, tok_raw, err) || !read_bytes(mask_path, mask_raw, err)) {
        fprintf(stderr, "%s\n", err.c_str());
        return 1;
    }
    if (tok_raw.size() != mask_raw.size() || tok_raw.empty() || tok_raw.size() % sizeof(int32_t)) {
        fprintf(stderr, "tok/mask size mismatch or invalid (tok=%zu mask=%zu)\n", tok_raw.size(),
                mask_raw.size());
        return 1;
    }
    const size_t n = tok_raw.size() / sizeof(int32_t);
    std::vector<int32_t> ids(n), mask(n);
    std::memcpy(ids.data(), tok_raw.data(), tok_raw.size());
    std::memcpy(mask.data(), mask_raw.data(), mask_raw.size());

    std::vector<float> emb;
    if (!enc.encode(ids.data(), (int)n, mask.data(), emb)) {
        fprintf(stderr, "encode failed: %s\n", enc.last_error().c_str());
        return 1;
    }
    if (!out_path.empty()) {
        if (!write_bytes(out_path, emb.data(), sizeof(float) * emb.size(), err)) {
            fprintf(stderr, "%s\n", err.c_str());
            return 1;
        }
        fprintf(stderr, "wrote text embedding (%zu floats) to %s\n", emb.size(), out_path.c_str());
    } else {
        fprintf(stdout, "text_embed[%zu]:\n", emb.size());
        for (size_t i = 0; i < std::min<size_t>(emb.size(), 8); ++i)
            fprintf(stdout, "  [%zu]=%g\n", i, emb[i]);
    }
    return 0;
}
