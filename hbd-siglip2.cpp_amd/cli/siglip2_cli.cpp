// siglip2-cli -- the vision encoder from the command line, over the
// drop-in classes (include/siglip2_vision.h, siglip2_preproc.h) on libs2x.
//
// Same arguments, raw-file contract and exit codes as the reference's
// src/siglip2_cli.cpp:16-29 (usage) and :58-207 (parsing, checks, output):
//   --model GGUF, and exactly one of
//   --pixel-values FILE   raw fp32 [n_patches, channels * patch^2]
//                         (--n-patches N, --shape H,W; default the native
//                         square grid of the model)
//   --image FILE          decoded by the caller in the reference's build
//                         (stb_image); not built here, so preprocess fails
//                         with a message, as preprocess_image_file does
//   --rgb FILE --rgb-shape H,W   raw interleaved u8 RGB of an H x W image,
//                         preprocessed on the GPU (the NaFlex front end,
//                         --max-num-patches as for --image)
//   --pooling probe|mean, --out FILE (raw fp32), else the first 8 and last 4
//   values as text on stdout.
// Exit codes: 0 ok, 1 load / read / encode failure, 2 bad arguments.
#include "siglip2_preproc.h"
#include "siglip2_vision.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

namespace {

void usage(const char *argv0) {
    fprintf(stderr,
            "siglip2-cli (vision encoder, libs2x on gfx950)\n"
            "\n"
            "Usage: %s --model <path.gguf> [--pixel-values <bin>|--image <img>|--rgb <raw>] [opts]\n"
            "\n"
            "  --model            GGUF file from scripts/convert_siglip2_to_gguf.py\n"
            "  --pixel-values     raw fp32 buffer of shape [n_patches, num_channels*patch_size^2]\n"
            "  --n-patches        with --pixel-values: number of patches in the buffer\n"
            "  --shape H,W        spatial patch grid (rows, cols); defaults to native square\n"
            "  --image            image file: needs an image decoder, not built here\n"
            "  --rgb              raw u8 RGB pixels (H*W*3 bytes), with --rgb-shape H,W\n"
            "  --max-num-patches  with --image / --rgb: cap on patches (default 256)\n"
            "  --pooling          'probe' (default; matches HF pooler_output) or 'mean'\n"
            "  --out              write embedding to this file as raw fp32; default: stdout text\n",
            argv0);
}

bool read_file(const std::string &path, std::vector<uint8_t> &out, std::string &err) {
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

bool write_file(const std::string &path, const void *data, size_t bytes, std::string &err) {
    std::ofstream f(path, std::ios::binary);
    if (!f) {
        err = "could not write: " + path;
        return false;
    }
    f.write(reinterpret_cast<const char *>(data), (std::streamsize)bytes);
    if (!f.good()) err = "could not write: " + path;
    return f.good();
}

// "H,W" -> two positive ints
bool parse_pair(const char *s, int &a, int &b) {
    const char *comma = strchr(s, ',');
    if (!comma) return false;
    a = std::atoi(std::string(s, comma).c_str());
    b = std::atoi(comma + 1);
    return true;
}

}  // namespace

int main(int argc, char **argv) {
    std::string model_path, pixel_path, image_path, rgb_path, out_path, pooling_str = "probe";
    int n_patches = -1, n_h = -1, n_w = -1, rgb_h = -1, rgb_w = -1, max_num_patches = 256;
    for (int i = 1; i < argc; ++i) {
        const bool more = i + 1 < argc;
        if ((!strcmp(argv[i], "--model") || !strcmp(argv[i], "-m")) && more) {
            model_path = argv[++i];
        } else if (!strcmp(argv[i], "--pixel-values") && more) {
            pixel_path = argv[++i];
        } else if (!strcmp(argv[i], "--image") && more) {
            image_path = argv[++i];
        } else if (!strcmp(argv[i], "--rgb") && more) {
            rgb_path = argv[++i];
        } else if (!strcmp(argv[i], "--rgb-shape") && more) {
            if (!parse_pair(argv[++i], rgb_h, rgb_w)) {
                fprintf(stderr, "--rgb-shape expects H,W (got: %s)\n", argv[i]);
                return 2;
            }
        } else if (!strcmp(argv[i], "--max-num-patches") && more) {
            max_num_patches = std::atoi(argv[++i]);
        } else if (!strcmp(argv[i], "--n-patches") && more) {
            n_patches = std::atoi(argv[++i]);
        } else if (!strcmp(argv[i], "--shape") && more) {
            if (!parse_pair(argv[++i], n_h, n_w)) {
                fprintf(stderr, "--shape expects H,W (got: %s)\n", argv[i]);
                return 2;
            }
        } else if (!strcmp(argv[i], "--pooling") && more) {
            pooling_str = argv[++i];
        } else if (!strcmp(argv[i], "--out") && more) {
            out_path = argv[++i];
        } else if (!strcmp(argv[i], "--help") || !strcmp(argv[i], "-h")) {
            usage(argv[0]);
            return 0;
        } else {
            fprintf(stderr, "Unknown arg: %s\n", argv[i]);
            usage(argv[0]);
            return 2;
        }
    }

    siglip2::Pooling pooling;
    if (pooling_str == "mean") {
        pooling = siglip2::Pooling::MEAN;
    } else if (pooling_str == "probe") {
        pooling = siglip2::Pooling::PROBE;
    } else {
        fprintf(stderr, "Unknown --pooling: %s (use 'probe' or 'mean')\n", pooling_str.c_str());
        return 2;
    }
    const int n_inputs = !pixel_path.empty() + !image_path.empty() + !rgb_path.empty();
    if (model_path.empty() || n_inputs != 1) {
        fprintf(stderr, "must supply --model and exactly one of --image / --pixel-values / --rgb\n");
        usage(argv[0]);
        return 2;
    }
    if (!rgb_path.empty() && (rgb_h <= 0 || rgb_w <= 0)) {
        fprintf(stderr, "--rgb needs --rgb-shape H,W\n");
        return 2;
    }

    siglip2::VisionEncoder enc;
    if (!enc.load(model_path)) {
        fprintf(stderr, "load failed: %s\n", enc.last_error().c_str());
        return 1;
    }
    const siglip2::VisionConfig &cfg = enc.config();
    const int feat = cfg.num_channels * cfg.patch_size * cfg.patch_size;

    std::string err;
    std::vector<float> pixels;
    float mean[3] = {0.5f, 0.5f, 0.5f}, std_v[3] = {0.5f, 0.5f, 0.5f};
    if (!image_path.empty() || !rgb_path.empty()) {
        siglip2::PreprocResult pp;
        bool ok;
        if (!image_path.empty()) {
            ok = siglip2::preprocess_image_file(image_path, max_num_patches, cfg.patch_size,
                                                1.0f / 255.0f, mean, std_v, pp, err);
        } else {
            std::vector<uint8_t> rgb;
            if (!read_file(rgb_path, rgb, err)) {
                fprintf(stderr, "%s\n", err.c_str());
                return 1;
            }
            if (rgb.size() != (size_t)rgb_h * rgb_w * 3) {
                fprintf(stderr, "rgb buffer size mismatch: got %zu bytes, expected %zu (%dx%dx3)\n",
                        rgb.size(), (size_t)rgb_h * rgb_w * 3, rgb_h, rgb_w);
                return 1;
            }
            ok = siglip2::preprocess_image_rgb(rgb.data(), rgb_h, rgb_w, max_num_patches,
                                               cfg.patch_size, 1.0f / 255.0f, mean, std_v, pp, err);
        }
        if (!ok) {
            fprintf(stderr, "preprocess failed: %s\n", err.c_str());
            return 1;
        }
        pixels = std::move(pp.pixel_values);
        n_h = pp.n_patches_h;
        n_w = pp.n_patches_w;
        fprintf(stderr, "preprocessed: grid=%dx%d (%d patches, max=%d)\n", n_h, n_w, n_h * n_w,
                max_num_patches);
    } else {
        if (n_h < 0 && n_w < 0) {
            const int side = (int)std::lround(std::sqrt((double)cfg.num_patches));
            n_h = n_w = side;
        } else if (n_h <= 0 || n_w <= 0) {
            fprintf(stderr, "--shape must specify both H and W\n");
            return 2;
        }
        if (n_patches < 0) n_patches = n_h * n_w;
        if (n_patches != n_h * n_w) {
            fprintf(stderr, "--n-patches=%d disagrees with --shape %d,%d (=%d).\n", n_patches, n_h,
                    n_w, n_h * n_w);
            return 2;
        }
        std::vector<uint8_t> raw;
        if (!read_file(pixel_path, raw, err)) {
            fprintf(stderr, "%s\n", err.c_str());
            return 1;
        }
        const size_t expected = sizeof(float) * (size_t)n_patches * feat;
        if (raw.size() != expected) {
            fprintf(stderr,
                    "pixel buffer size mismatch: got %zu bytes, expected %zu (n_patches=%d feat=%d)\n",
                    raw.size(), expected, n_patches, feat);
            return 1;
        }
        pixels.resize(raw.size() / sizeof(float));
        std::memcpy(pixels.data(), raw.data(), raw.size());
    }

    std::vector<float> emb;
    if (!enc.encode(pixels.data(), n_h, n_w, pooling, emb)) {
        fprintf(stderr, "encode failed: %s\n", enc.last_error().c_str());
        return 1;
    }
    if (!out_path.empty()) {
        if (!write_file(out_path, emb.data(), sizeof(float) * emb.size(), err)) {
            fprintf(stderr, "%s\n", err.c_str());
            return 1;
        }
        fprintf(stderr, "wrote embedding (%zu floats) to %s\n", emb.size(), out_path.c_str());
    } else {
        fprintf(stdout, "embedding[%zu]:\n", emb.size());
        for (size_t i = 0; i < std::min<size_t>(emb.size(), 8); ++i)
            fprintf(stdout, "  [%zu]=%g\n", i, emb[i]);
        if (emb.size() > 16) {
            fprintf(stdout, "  ...\n");
            for (size_t i = emb.size() - 4; i < emb.size(); ++i) fprintf(stdout, "  [%zu]=%g\n", i, emb[i]);
        }
    }
    return 0;
}
