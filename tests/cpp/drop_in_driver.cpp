// drop_in_driver.cpp -- runs the reference-shaped C++ classes of libs2x
// (siglip2::VisionEncoder, siglip2::TextEncoder, siglip2::preprocess_image_rgb,
// include/siglip2_*.h) as a program compiled against those headers would:
// inputs and outputs are raw little-endian files, errors go to stderr with a
// non-zero exit code.  The GPU tests compare its outputs with the C-ABI's.
//
//   drop_in_driver vision  <gguf> <pixels.f32> <n_h> <n_w> <0 mean | 1 probe> <out.f32>
//   drop_in_driver text    <gguf> <ids.i32> <n_tok> <n_batch> <out.f32>
//   drop_in_driver preproc <rgb.u8> <h> <w> <max_patches> <out.f32>
//   drop_in_driver badload <path>      (expects load() to fail with a message)
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iterator>
#include <string>
#include <vector>

#include "siglip2_preproc.h"
#include "siglip2_text.h"
#include "siglip2_vision.h"

namespace {

template <class T>
bool read_file(const char *path, std::vector<T> &out) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    std::vector<char> bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    out.resize(bytes.size() / sizeof(T));
    std::memcpy(out.data(), bytes.data(), out.size() * sizeof(T));
    return true;
}

template <class T>
bool write_file(const char *path, const std::vector<T> &v) {
    std::ofstream f(path, std::ios::binary);
    f.write(reinterpret_cast<const char *>(v.data()), (std::streamsize)(v.size() * sizeof(T)));
    return (bool)f;
}

int die(const std::string &msg) {
    std::fprintf(stderr, "drop_in_driver: %s\n", msg.c_str());
    return 1;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc < 3) return die("usage: drop_in_driver vision|text|preproc|badload ...");
    const std::string mode = argv[1];
    if (mode == "vision" && argc == 8) {
        siglip2::VisionEncoder enc;
        if (!enc.load(argv[2])) return die("load: " + enc.last_error());
        std::vector<float> px, out;
        if (!read_file(argv[3], px)) return die("cannot read pixels");
        const int n_h = std::atoi(argv[4]), n_w = std::atoi(argv[5]);
        const siglip2::Pooling pool = std::atoi(argv[6]) ? siglip2::Pooling::PROBE : siglip2::Pooling::MEAN;
        const size_t row = (size_t)enc.config().num_channels * enc.config().patch_size *
                           enc.config().patch_size;
        if (px.size() != row * (size_t)(n_h * n_w)) return die("pixel file size");
        if (!enc.encode(px.data(), n_h, n_w, pool, out)) return die("encode: " + enc.last_error());
        if ((int)out.size() != enc.config().hidden_size) return die("embedding size");
        return write_file(argv[7], out) ? 0 : die("cannot write output");
    }
    if (mode == "text" && argc == 7) {
        siglip2::TextEncoder enc;
        if (!enc.load(argv[2])) return die("load: " + enc.last_error());
        std::vector<int32_t> ids;
        std::vector<float> out;
        if (!read_file(argv[3], ids)) return die("cannot read ids");
        const int n_tok = std::atoi(argv[4]), n_batch = std::atoi(argv[5]);
        if ((int)ids.size() != n_tok * n_batch) return die("ids file size");
        if (n_batch == 1) {
            if (!enc.encode(ids.data(), n_tok, nullptr, out)) return die("encode: " + enc.last_error());
        } else {
            // the reference rejects a mask for batches: so must the drop-in
            std::vector<int32_t> mask(ids.size(), 1);
            std::vector<float> dummy;
            if (enc.encode_batch(ids.data(), n_tok, n_batch, mask.data(), dummy))
                return die("encode_batch accepted a mask");
            if (!enc.encode_batch(ids.data(), n_tok, n_batch, nullptr, out))
                return die("encode_batch: " + enc.last_error());
        }
        return write_file(argv[6], out) ? 0 : die("cannot write output");
    }
    if (mode == "preproc" && argc == 7) {
        std::vector<uint8_t> rgb;
        if (!read_file(argv[2], rgb)) return die("cannot read rgb");
        const int h = std::atoi(argv[3]), w = std::atoi(argv[4]), mp = std::atoi(argv[5]);
        if ((int64_t)rgb.size() != (int64_t)h * w * 3) return die("rgb file size");
        float mean[3] = {0.5f, 0.5f, 0.5f}, std_[3] = {0.5f, 0.5f, 0.5f};
        siglip2::PreprocResult res;
        std::string err;
        if (!siglip2::preprocess_image_rgb(rgb.data(), h, w, mp, 16, 1.0f / 255.0f, mean, std_, res, err))
            return die("preprocess: " + err);
        std::printf("%d %d\n", res.n_patches_h, res.n_patches_w);
        return write_file(argv[6], res.pixel_values) ? 0 : die("cannot write output");
    }
    if (mode == "badload" && argc == 3) {
        siglip2::VisionEncoder enc;
        if (enc.load(argv[2])) return die("load of a bad file succeeded");
        if (enc.last_error().empty()) return die("no error message");
        std::printf("%s\n", enc.last_error().c_str());
        return 0;
    }
    return die("bad arguments for mode " + mode);
}
