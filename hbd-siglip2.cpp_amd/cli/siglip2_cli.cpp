// siglip2-cli -- the vision encoder from the command line, over the
// drop-in classes (include/siglip2_vision.h, siglip2_preproc.h) on libs2x.
//
// The flags, exit codes and messages are those of the reference's
// src/siglip2_cli.cpp (its command-line contract):
//   --model GGUF, and exactly one input:
//     --pixel-values FILE   raw fp32 [n_patches, channels * patch^2]
//                           (--n-patches N, --shape H,W; without --shape the
//                           model's native square grid)
//     --image FILE          needs an image decoder, which this build does
//                           not have: preprocessing fails with a message
//     --rgb FILE --rgb-shape H,W   raw interleaved u8 RGB of an H x W image,
//                           preprocessed on the GPU (NaFlex, capped by
//                           --max-num-patches)
//   --pooling probe|mean, --out FILE (raw fp32), else a summary on stdout.
// Exit codes: 0 ok, 1 load / read / preprocess / encode failure, 2 bad
// arguments.
#include "cli_common.h"
#include "siglip2_preproc.h"
#include "siglip2_vision.h"

#include <cmath>
#include <cstdio>
#include <string>
#include <vector>

namespace {

using namespace s2xcli;

struct Request {
    std::string model, pixel_file, image_file, rgb_file, out_file, pooling = "probe";
    int n_patches = -1;
    int grid[2] = {-1, -1};      // --shape
    int rgb_grid[2] = {-1, -1};  // --rgb-shape
    int max_patches = 256;
};

std::vector<Option> options(Request &r) {
    std::vector<Option> t;
    auto text = [&](const char *n, const char *a, const char *m, const char *h, std::string *s) {
        Option o{n, a, m, h};
        o.text = s;
        t.push_back(o);
    };
    auto number = [&](const char *n, const char *m, const char *h, int *v) {
        Option o{n, nullptr, m, h};
        o.number = v;
        t.push_back(o);
    };
    auto grid = [&](const char *n, const char *h, int *g) {
        Option o{n, nullptr, "H,W", h};
        o.grid = g;
        t.push_back(o);
    };
    text("--model", "-m", "<path.gguf>", "GGUF file of the reference converter", &r.model);
    text("--pixel-values", nullptr, "<file>", "raw fp32 [n_patches, channels*patch^2]", &r.pixel_file);
    number("--n-patches", "<n>", "patches in the --pixel-values file", &r.n_patches);
    grid("--shape", "patch grid of --pixel-values (default: native square)", r.grid);
    text("--image", nullptr, "<file>", "image file (needs a decoder: not in this build)", &r.image_file);
    text("--rgb", nullptr, "<file>", "raw u8 RGB, H*W*3 bytes (with --rgb-shape)", &r.rgb_file);
    grid("--rgb-shape", "height and width of the --rgb image", r.rgb_grid);
    number("--max-num-patches", "<n>", "patch cap for --image / --rgb (default 256)", &r.max_patches);
    text("--pooling", nullptr, "probe|mean", "probe (default, HF pooler_output) or mean", &r.pooling);
    text("--out", nullptr, "<file>", "raw fp32 embedding (default: summary on stdout)", &r.out_file);
    return t;
}

void usage(const std::vector<Option> &table, const char *prog) {
    print_usage(stderr, "siglip2-cli (vision encoder, libs2x on gfx950)",
                {std::string(prog) + " --model <path.gguf> [--pixel-values <bin>|--image <img>|--rgb <raw>] [opts]"},
                table);
}

// Argument checks that need no model; 0 or the exit code.
int check(const Request &r, siglip2::Pooling &pooling) {
    if (r.pooling == "probe") {
        pooling = siglip2::Pooling::PROBE;
    } else if (r.pooling == "mean") {
        pooling = siglip2::Pooling::MEAN;
    } else {
        std::fprintf(stderr, "Unknown --pooling: %s (use 'probe' or 'mean')\n", r.pooling.c_str());
        return EXIT_USAGE;
    }
    const int inputs = (int)!r.pixel_file.empty() + (int)!r.image_file.empty() + (int)!r.rgb_file.empty();
    if (r.model.empty() || inputs != 1) {
        std::fprintf(stderr, "must supply --model and exactly one of --image / --pixel-values / --rgb\n");
        return EXIT_USAGE;
    }
    if (!r.rgb_file.empty() && (r.rgb_grid[0] <= 0 || r.rgb_grid[1] <= 0)) {
        std::fprintf(stderr, "--rgb needs --rgb-shape H,W\n");
        return EXIT_USAGE;
    }
    return 0;
}

struct Patches {
    std::vector<float> values;
    int n_h = 0, n_w = 0;
};

// --pixel-values: the grid from --shape / --n-patches / the model, then the
// file of exactly that many patch rows
int pixel_input(const Request &r, const siglip2::VisionConfig &cfg, Patches &p) {
    int n_h = r.grid[0], n_w = r.grid[1];
    if (n_h < 0 && n_w < 0) {
        n_h = n_w = (int)std::lround(std::sqrt((double)cfg.num_patches));
    } else if (n_h <= 0 || n_w <= 0) {
        std::fprintf(stderr, "--shape must specify both H and W\n");
        return EXIT_USAGE;
    }
    const int count = r.n_patches < 0 ? n_h * n_w : r.n_patches;
    if (count != n_h * n_w) {
        std::fprintf(stderr, "--n-patches=%d disagrees with --shape %d,%d (=%d).\n", count, n_h, n_w,
                     n_h * n_w);
        return EXIT_USAGE;
    }
    const size_t row = (size_t)cfg.num_channels * cfg.patch_size * cfg.patch_size;
    std::vector<uint8_t> bytes;
    std::string err;
    if (!slurp(r.pixel_file, bytes, err)) {
        std::fprintf(stderr, "%s\n", err.c_str());
        return EXIT_FAIL;
    }
    const size_t want = (size_t)count * row * sizeof(float);
    if (bytes.size() != want) {
        std::fprintf(stderr, "pixel buffer size mismatch: got %zu bytes, expected %zu (n_patches=%d feat=%zu)\n",
                     bytes.size(), want, count, row);
        return EXIT_FAIL;
    }
    p.values = as_values<float>(bytes);
    p.n_h = n_h;
    p.n_w = n_w;
    return 0;
}

// --image / --rgb: the NaFlex front end (rescale 1/255, mean = std = 0.5)
int image_input(const Request &r, const siglip2::VisionConfig &cfg, Patches &p) {
    float mean[3] = {0.5f, 0.5f, 0.5f}, stdv[3] = {0.5f, 0.5f, 0.5f};  // the interface takes float*
    siglip2::PreprocResult pre;
    std::string err;
    bool ok;
    if (!r.rgb_file.empty()) {
        std::vector<uint8_t> rgb;
        if (!slurp(r.rgb_file, rgb, err)) {
            std::fprintf(stderr, "%s\n", err.c_str());
            return EXIT_FAIL;
        }
        const size_t want = (size_t)r.rgb_grid[0] * r.rgb_grid[1] * 3;
        if (rgb.size() != want) {
            std::fprintf(stderr, "rgb buffer size mismatch: got %zu bytes, expected %zu (%dx%dx3)\n",
                         rgb.size(), want, r.rgb_grid[0], r.rgb_grid[1]);
            return EXIT_FAIL;
        }
        ok = siglip2::preprocess_image_rgb(rgb.data(), r.rgb_grid[0], r.rgb_grid[1], r.max_patches,
                                           cfg.patch_size, 1.0f / 255.0f, mean, stdv, pre, err);
    } else {
        ok = siglip2::preprocess_image_file(r.image_file, r.max_patches, cfg.patch_size, 1.0f / 255.0f,
                                            mean, stdv, pre, err);
    }
    if (!ok) {
        std::fprintf(stderr, "preprocess failed: %s\n", err.c_str());
        return EXIT_FAIL;
    }
    p.values = std::move(pre.pixel_values);
    p.n_h = pre.n_patches_h;
    p.n_w = pre.n_patches_w;
    std::fprintf(stderr, "preprocessed: grid=%dx%d (%d patches, max=%d)\n", p.n_h, p.n_w, p.n_h * p.n_w,
                 r.max_patches);
    return 0;
}

int run(const Request &r, siglip2::Pooling pooling) {
    siglip2::VisionEncoder enc;
    if (!enc.load(r.model)) {
        std::fprintf(stderr, "load failed: %s\n", enc.last_error().c_str());
        return EXIT_FAIL;
    }
    Patches p;
    const int rc = r.pixel_file.empty() ? image_input(r, enc.config(), p) : pixel_input(r, enc.config(), p);
    if (rc) return rc;
    std::vector<float> emb;
    if (!enc.encode(p.values.data(), p.n_h, p.n_w, pooling, emb)) {
        std::fprintf(stderr, "encode failed: %s\n", enc.last_error().c_str());
        return EXIT_FAIL;
    }
    if (r.out_file.empty()) {
        print_summary(stdout, "embedding", emb);
        return EXIT_OK;
    }
    std::string err;
    if (!spill(r.out_file, emb.data(), emb.size() * sizeof(float), err)) {
        std::fprintf(stderr, "%s\n", err.c_str());
        return EXIT_FAIL;
    }
    std::fprintf(stderr, "wrote embedding (%zu floats) to %s\n", emb.size(), r.out_file.c_str());
    return EXIT_OK;
}

}  // namespace

int main(int argc, char **argv) {
    Request req;
    const std::vector<Option> table = options(req);
    std::string err;
    switch (parse(argc, argv, table, err)) {
    case Parsed::help:
        usage(table, argv[0]);
        return EXIT_OK;
    case Parsed::bad:
        std::fprintf(stderr, "%s\n", err.c_str());
        if (err.rfind("Unknown arg", 0) == 0) usage(table, argv[0]);
        return EXIT_USAGE;
    case Parsed::ok:
        break;
    }
    siglip2::Pooling pooling = siglip2::Pooling::PROBE;
    const int rc = check(req, pooling);
    if (rc) {
        if (rc == EXIT_USAGE && req.model.empty()) usage(table, argv[0]);
        return rc;
    }
    return run(req, pooling);
}
