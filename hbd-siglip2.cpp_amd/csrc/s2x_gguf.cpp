// s2x_gguf.cpp -- GGUF reader for siglip2 weight files (host only).
//
// Replaces the reference's GGUF path into the encoders
// (src/gguf_loader.cpp:205-337 tensor upload, src/siglip2_vision.cpp:424-560
// and src/siglip2_text.cpp:424-540 tensor binding): the file is mapped
// read-only, its metadata and tensor directory parsed, and the tensors bound
// by the converter's names (scripts/convert_siglip2_to_gguf.py:7-35) into
// s2x_vision_weights / s2x_text_weights.  Q8_0 and F32 tensors are used in
// place; F16 vectors are widened to F32.  ffn_down matrices stored as F16
// -- what the converter writes for them in a q8_0 file, K = 4304 not being a
// multiple of 32 (scripts/convert_siglip2_to_gguf.py:241-290) -- stay F16
// and run as F16 x F32 products, as the reference's encoders keep the
// on-disk type (src/siglip2_vision.cpp:496-556, dup_meta).  Any other F16 /
// F32 matrix (a file converted to f16 or f32 throughout) is quantized to
// Q8_0 on load (ggml's quantize_row_q8_0_ref rule, K zero-padded to a
// multiple of 32), where the reference would multiply in F16 / F32: this
// library's GEMMs for those matrices are the Q8_0 ones.
//
// File layout (GGUF v2/v3): magic "GGUF", u32 version, u64 tensor count,
// u64 metadata count; metadata entries (string key, u32 type, value);
// tensor infos (string name, u32 n_dims, u64 ne[n_dims], u32 ggml type,
// u64 offset); padding to general.alignment (default 32); tensor data.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "s2x.h"
#include "s2x_internal.h"

using namespace s2x;

namespace {

enum GgufType : uint32_t {
    GT_U8 = 0, GT_I8 = 1, GT_U16 = 2, GT_I16 = 3, GT_U32 = 4, GT_I32 = 5, GT_F32 = 6,
    GT_BOOL = 7, GT_STRING = 8, GT_ARRAY = 9, GT_U64 = 10, GT_I64 = 11, GT_F64 = 12,
};
enum GgmlType : uint32_t { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8 };

struct Scalar {
    uint32_t type = 0;
    uint64_t u = 0;   // integer types and bool
    int64_t i = 0;
    double f = 0.0;   // float types
};

struct TensorInfo {
    std::string name;
    uint32_t type = 0;
    std::vector<int64_t> ne;
    uint64_t offset = 0;
    const uint8_t *data = nullptr;
    int64_t nelem() const {
        int64_t n = 1;
        for (int64_t e : ne) n *= e;
        return n;
    }
};

float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {  // subnormal: normalise
            int e = -1;
            uint32_t m = man;
            do {
                ++e;
                m <<= 1;
            } while ((m & 0x400) == 0);
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((m & 0x3ff) << 13);
        }
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// IEEE binary16, round to nearest even (overflow -> inf)
uint16_t float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000;
    const uint32_t ax = x & 0x7fffffff;
    if (ax >= 0x7f800000) return (uint16_t)(sign | 0x7c00 | (ax > 0x7f800000 ? 0x200 : 0));
    if (ax >= 0x477ff000) return (uint16_t)(sign | 0x7c00);  // rounds past 65504
    if (ax < 0x38800000) {  // subnormal or zero in half
        if (ax < 0x33000000) return (uint16_t)sign;
        const uint32_t m = (ax & 0x7fffff) | 0x800000;
        const int shift = 126 - (int)(ax >> 23);  // 14..24
        const uint32_t q = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        uint32_t r = q + ((rem > half || (rem == half && (q & 1))) ? 1 : 0);
        return (uint16_t)(sign | r);
    }
    uint32_t r = ax + 0xfff + ((ax >> 13) & 1);  // round to nearest even at bit 13
    r -= 0x38000000;
    return (uint16_t)(sign | (r >> 13));
}

// ggml quantize_row_q8_0_ref: d = amax/127, id = d ? 1/d : 0, q = roundf(x*id)
void quantize_row_q8_0(const float *x, int64_t K, int64_t K_pad, uint8_t *out) {
    for (int64_t b = 0; b < K_pad / 32; ++b) {
        float v[32];
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const int64_t k = b * 32 + j;
            v[j] = k < K ? x[k] : 0.0f;
            amax = std::fmax(amax, std::fabs(v[j]));
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t *blk = out + b * 34;
        const uint16_t dh = float_to_half(d);
        std::memcpy(blk, &dh, 2);
        for (int j = 0; j < 32; ++j) blk[2 + j] = (uint8_t)(int8_t)std::roundf(v[j] * id);
    }
}

}  // namespace

struct s2x_gguf {
    void *map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    std::map<std::string, Scalar> kv;
    std::map<std::string, TensorInfo> tensors;
    std::vector<std::unique_ptr<uint8_t[]>> owned;  // converted tensors
    std::vector<s2x_layer_weights> vision_layers, text_layers;

    ~s2x_gguf() {
        if (map && map != MAP_FAILED) munmap(map, size);
    }

    uint8_t *own(size_t bytes) {
        owned.emplace_back(new uint8_t[bytes]);
        return owned.back().get();
    }
};

namespace {

struct Reader {
    const uint8_t *p, *end;
    bool ok = true;
    template <class T> T get() {
        T v{};
        if ((size_t)(end - p) < sizeof(T)) {
            ok = false;
            return v;
        }
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str(uint32_t version) {
        const uint64_t n = version == 1 ? get<uint32_t>() : get<uint64_t>();
        if (!ok || n > (uint64_t)(end - p)) {
            ok = false;
            return {};
        }
        std::string s(reinterpret_cast<const char *>(p), (size_t)n);
        p += n;
        return s;
    }
    bool skip(uint64_t n) {
        if (n > (uint64_t)(end - p)) return ok = false;
        p += n;
        return true;
    }
};

size_t scalar_size(uint32_t t) {
    switch (t) {
    case GT_U8: case GT_I8: case GT_BOOL: return 1;
    case GT_U16: case GT_I16: return 2;
    case GT_U32: case GT_I32: case GT_F32: return 4;
    case GT_U64: case GT_I64: case GT_F64: return 8;
    default: return 0;
    }
}

bool read_scalar(Reader &r, uint32_t t, Scalar &s) {
    s.type = t;
    switch (t) {
    case GT_U8: s.u = r.get<uint8_t>(); break;
    case GT_I8: s.i = r.get<int8_t>(); s.u = (uint64_t)s.i; break;
    case GT_U16: s.u = r.get<uint16_t>(); break;
    case GT_I16: s.i = r.get<int16_t>(); s.u = (uint64_t)s.i; break;
    case GT_U32: s.u = r.get<uint32_t>(); break;
    case GT_I32: s.i = r.get<int32_t>(); s.u = (uint64_t)s.i; break;
    case GT_U64: s.u = r.get<uint64_t>(); break;
    case GT_I64: s.i = r.get<int64_t>(); s.u = (uint64_t)s.i; break;
    case GT_BOOL: s.u = r.get<uint8_t>(); break;
    case GT_F32: s.f = r.get<float>(); break;
    case GT_F64: s.f = r.get<double>(); break;
    default: return false;
    }
    if (t == GT_U8 || t == GT_U16 || t == GT_U32 || t == GT_U64 || t == GT_BOOL) s.i = (int64_t)s.u;
    if (t != GT_F32 && t != GT_F64) s.f = (double)s.i;
    return r.ok;
}

int parse(s2x_gguf *g) {
    Reader r{reinterpret_cast<const uint8_t *>(g->map),
             reinterpret_cast<const uint8_t *>(g->map) + g->size};
    if (r.get<uint32_t>() != 0x46554747u) return fail(S2X_ERR_INVALID_ARG, "gguf: bad magic");
    g->version = r.get<uint32_t>();
    if (g->version < 1 || g->version > 3)
        return fail(S2X_ERR_UNSUPPORTED, "gguf: version %u not supported", g->version);
    const uint64_t n_tensors = g->version == 1 ? r.get<uint32_t>() : r.get<uint64_t>();
    const uint64_t n_kv = g->version == 1 ? r.get<uint32_t>() : r.get<uint64_t>();
    if (!r.ok || n_tensors > (1u << 24) || n_kv > (1u << 24))
        return fail(S2X_ERR_INVALID_ARG, "gguf: truncated header");
    for (uint64_t i = 0; i < n_kv; ++i) {
        const std::string key = r.str(g->version);
        const uint32_t t = r.get<uint32_t>();
        if (!r.ok) return fail(S2X_ERR_INVALID_ARG, "gguf: truncated metadata");
        if (t == GT_STRING) {
            r.str(g->version);
        } else if (t == GT_ARRAY) {
            const uint32_t et = r.get<uint32_t>();
            const uint64_t n = g->version == 1 ? r.get<uint32_t>() : r.get<uint64_t>();
            if (et == GT_STRING) {
                for (uint64_t j = 0; j < n && r.ok; ++j) r.str(g->version);
            } else {
                const size_t es = scalar_size(et);
                if (es == 0 || n > (uint64_t)(r.end - r.p) / es)
                    return fail(S2X_ERR_INVALID_ARG, "gguf: bad array in '%s'", key.c_str());
                r.skip(n * es);
            }
        } else {
            Scalar s;
            if (!read_scalar(r, t, s))
                return fail(S2X_ERR_INVALID_ARG, "gguf: bad value type %u for '%s'", t, key.c_str());
            g->kv[key] = s;
        }
        if (!r.ok) return fail(S2X_ERR_INVALID_ARG, "gguf: truncated metadata");
    }
    std::vector<TensorInfo> infos;
    for (uint64_t i = 0; i < n_tensors; ++i) {
        TensorInfo ti;
        ti.name = r.str(g->version);
        const uint32_t nd = r.get<uint32_t>();
        if (!r.ok || nd == 0 || nd > 4) return fail(S2X_ERR_INVALID_ARG, "gguf: bad tensor info");
        for (uint32_t d = 0; d < nd; ++d)
            ti.ne.push_back(g->version == 1 ? (int64_t)r.get<uint32_t>() : (int64_t)r.get<uint64_t>());
        ti.type = r.get<uint32_t>();
        ti.offset = r.get<uint64_t>();
        if (!r.ok) return fail(S2X_ERR_INVALID_ARG, "gguf: truncated tensor directory");
        for (int64_t e : ti.ne)
            if (e <= 0) return fail(S2X_ERR_INVALID_ARG, "gguf: tensor '%s' has a bad shape", ti.name.c_str());
        infos.push_back(std::move(ti));
    }
    uint64_t align = 32;
    auto it = g->kv.find("general.alignment");
    if (it != g->kv.end()) align = it->second.u;
    if (align == 0 || (align & (align - 1))) return fail(S2X_ERR_INVALID_ARG, "gguf: bad alignment");
    const uint64_t hdr = (uint64_t)(r.p - reinterpret_cast<const uint8_t *>(g->map));
    const uint64_t data0 = (hdr + align - 1) / align * align;
    for (auto &ti : infos) {
        uint64_t bytes;
        const int64_t n = ti.nelem();
        if (ti.type == T_F32) bytes = (uint64_t)n * 4;
        else if (ti.type == T_F16) bytes = (uint64_t)n * 2;
        else if (ti.type == T_Q8_0) {
            if (ti.ne[0] % 32) return fail(S2X_ERR_INVALID_ARG, "gguf: Q8_0 tensor '%s' with ne0 %% 32", ti.name.c_str());
            bytes = (uint64_t)n / 32 * 34;
        } else {
            bytes = 0;  // other types are rejected only if a bound tensor has one
        }
        if (data0 + ti.offset > g->size || bytes > g->size - data0 - ti.offset)
            return fail(S2X_ERR_INVALID_ARG, "gguf: tensor '%s' past the end of the file", ti.name.c_str());
        ti.data = reinterpret_cast<const uint8_t *>(g->map) + data0 + ti.offset;
        g->tensors[ti.name] = ti;
    }
    return S2X_OK;
}

int64_t kv_int(const s2x_gguf *g, const char *key, int64_t dflt) {
    auto it = g->kv.find(key);
    return it == g->kv.end() ? dflt : it->second.i;
}
double kv_float(const s2x_gguf *g, const char *key, double dflt) {
    auto it = g->kv.find(key);
    return it == g->kv.end() ? dflt : it->second.f;
}

// F32 vector of n values (F32 in place, F16 widened)
int bind_vec(s2x_gguf *g, const std::string &name, int64_t n, const float **out) {
    auto it = g->tensors.find(name);
    if (it == g->tensors.end()) return fail(S2X_ERR_INVALID_ARG, "gguf: missing tensor %s", name.c_str());
    const TensorInfo &t = it->second;
    if (t.nelem() != n)
        return fail(S2X_ERR_INVALID_ARG, "gguf: %s has %lld values, expected %lld", name.c_str(),
                    (long long)t.nelem(), (long long)n);
    if (t.type == T_F32) {
        if (reinterpret_cast<uintptr_t>(t.data) % 4 == 0) {
            *out = reinterpret_cast<const float *>(t.data);
            return S2X_OK;
        }
        float *f = reinterpret_cast<float *>(g->own((size_t)n * 4));
        std::memcpy(f, t.data, (size_t)n * 4);
        *out = f;
        return S2X_OK;
    }
    if (t.type == T_F16) {
        float *f = reinterpret_cast<float *>(g->own((size_t)n * 4));
        for (int64_t i = 0; i < n; ++i) {
            uint16_t h;
            std::memcpy(&h, t.data + 2 * i, 2);
            f[i] = half_to_float(h);
        }
        *out = f;
        return S2X_OK;
    }
    return fail(S2X_ERR_UNSUPPORTED, "gguf: %s has ggml type %u (F32/F16 expected)", name.c_str(), t.type);
}

// Q8_0 matrix ne = (K, N) with K padded to K_pad (a multiple of 32, K_pad - K < 32)
int bind_q8(s2x_gguf *g, const std::string &name, int64_t K, int64_t K_pad, int64_t N,
            const void **out) {
    auto it = g->tensors.find(name);
    if (it == g->tensors.end()) return fail(S2X_ERR_INVALID_ARG, "gguf: missing tensor %s", name.c_str());
    const TensorInfo &t = it->second;
    const int64_t ne0 = t.ne[0], ne1 = t.nelem() / t.ne[0];
    if (ne1 != N || (ne0 != K && ne0 != K_pad))
        return fail(S2X_ERR_INVALID_ARG, "gguf: %s has shape (%lld, %lld), expected (%lld|%lld, %lld)",
                    name.c_str(), (long long)ne0, (long long)ne1, (long long)K, (long long)K_pad,
                    (long long)N);
    if (t.type == T_Q8_0) {
        if (ne0 != K_pad)
            return fail(S2X_ERR_INVALID_ARG, "gguf: Q8_0 %s has K %lld, expected %lld", name.c_str(),
                        (long long)ne0, (long long)K_pad);
        *out = t.data;
        return S2X_OK;
    }
    if (t.type != T_F32 && t.type != T_F16)
        return fail(S2X_ERR_UNSUPPORTED, "gguf: %s has ggml type %u (Q8_0/F16/F32 expected)",
                    name.c_str(), t.type);
    uint8_t *q = g->own((size_t)(N * (K_pad / 32) * 34));
    std::vector<float> row((size_t)ne0);
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t k = 0; k < ne0; ++k) {
            if (t.type == T_F32) {
                std::memcpy(&row[(size_t)k], t.data + (n * ne0 + k) * 4, 4);
            } else {
                uint16_t h;
                std::memcpy(&h, t.data + (n * ne0 + k) * 2, 2);
                row[(size_t)k] = half_to_float(h);
            }
        }
        quantize_row_q8_0(row.data(), ne0, K_pad, q + n * (K_pad / 32) * 34);
    }
    *out = q;
    return S2X_OK;
}

// ffn_down: an F16 matrix (K = F in ne0) is used in place as F16 rows
// (*is_f16 = 1); Q8_0 / F32 go through bind_q8 (*is_f16 = 0).
int bind_down(s2x_gguf *g, const std::string &name, int64_t F, int64_t F_pad, int64_t N,
              const void **out, int *is_f16) {
    auto it = g->tensors.find(name);
    if (it == g->tensors.end()) return fail(S2X_ERR_INVALID_ARG, "gguf: missing tensor %s", name.c_str());
    const TensorInfo &t = it->second;
    if (t.type != T_F16) {
        *is_f16 = 0;
        return bind_q8(g, name, F, F_pad, N, out);
    }
    const int64_t ne0 = t.ne[0], ne1 = t.nelem() / t.ne[0];
    if (ne0 != F || ne1 != N)
        return fail(S2X_ERR_INVALID_ARG, "gguf: F16 %s has shape (%lld, %lld), expected (%lld, %lld)",
                    name.c_str(), (long long)ne0, (long long)ne1, (long long)F, (long long)N);
    if (reinterpret_cast<uintptr_t>(t.data) % 2 != 0) {
        uint8_t *c = g->own((size_t)(N * F * 2));
        std::memcpy(c, t.data, (size_t)(N * F * 2));
        *out = c;
    } else {
        *out = t.data;
    }
    *is_f16 = 1;
    return S2X_OK;
}

std::string blk(const char *tower, int il, const char *suffix) {
    return std::string(tower) + ".blk." + std::to_string(il) + "." + suffix;
}

// down_f16: set from the first layer's ffn_down; every other ffn_down of the
// tower must have the same type
int bind_layers(s2x_gguf *g, const char *tower, int64_t n_layer, int64_t H, int64_t F,
                int64_t F_pad, std::vector<s2x_layer_weights> &layers, int32_t *down_f16) {
    layers.assign((size_t)n_layer, s2x_layer_weights{});
    for (int64_t il = 0; il < n_layer; ++il) {
        s2x_layer_weights &L = layers[(size_t)il];
        const int i = (int)il;
        int st, f16 = 0;
        if ((st = bind_vec(g, blk(tower, i, "ln1.weight"), H, &L.ln1_w)) ||
            (st = bind_vec(g, blk(tower, i, "ln1.bias"), H, &L.ln1_b)) ||
            (st = bind_q8(g, blk(tower, i, "attn_qkv.weight"), H, H, 3 * H, &L.qkv_w)) ||
            (st = bind_vec(g, blk(tower, i, "attn_qkv.bias"), 3 * H, &L.qkv_b)) ||
            (st = bind_q8(g, blk(tower, i, "attn_o.weight"), H, H, H, &L.o_w)) ||
            (st = bind_vec(g, blk(tower, i, "attn_o.bias"), H, &L.o_b)) ||
            (st = bind_vec(g, blk(tower, i, "ln2.weight"), H, &L.ln2_w)) ||
            (st = bind_vec(g, blk(tower, i, "ln2.bias"), H, &L.ln2_b)) ||
            (st = bind_q8(g, blk(tower, i, "ffn_up.weight"), H, H, F, &L.up_w)) ||
            (st = bind_vec(g, blk(tower, i, "ffn_up.bias"), F, &L.up_b)) ||
            (st = bind_down(g, blk(tower, i, "ffn_down.weight"), F, F_pad, H, &L.down_w, &f16)) ||
            (st = bind_vec(g, blk(tower, i, "ffn_down.bias"), H, &L.down_b)))
            return st;
        if (il == 0) *down_f16 = f16;
        if (f16 != *down_f16)
            return fail(S2X_ERR_UNSUPPORTED, "gguf: %s ffn_down types differ between layers", tower);
    }
    return S2X_OK;
}

// K of ffn_down as stored: a Q8_0 tensor carries its padded K in ne0
int64_t ffn_down_kpad(const s2x_gguf *g, const char *tower, int64_t F) {
    const int64_t pad = (F + 31) / 32 * 32;
    auto it = g->tensors.find(blk(tower, 0, "ffn_down.weight"));
    if (it != g->tensors.end() && it->second.type == T_Q8_0) return it->second.ne[0];
    return pad;
}

}  // namespace

extern "C" {

int s2x_gguf_open(const char *path, s2x_gguf **out) {
    if (!path || !out) return fail(S2X_ERR_INVALID_ARG, "gguf_open: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(S2X_ERR_INVALID_ARG, "gguf_open: cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        return fail(S2X_ERR_INVALID_ARG, "gguf_open: %s is not a GGUF file", path);
    }
    std::unique_ptr<s2x_gguf> g(new s2x_gguf);
    g->size = (size_t)st.st_size;
    g->map = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (g->map == MAP_FAILED) {
        g->map = nullptr;
        return fail(S2X_ERR_OOM, "gguf_open: mmap of %s failed", path);
    }
    const int st2 = parse(g.get());
    if (st2 != S2X_OK) return st2;
    *out = g.release();
    return S2X_OK;
}

void s2x_gguf_close(s2x_gguf *g) { delete g; }

int s2x_gguf_vision_weights(s2x_gguf *g, s2x_vision_weights *w) {
    if (!g || !w) return fail(S2X_ERR_INVALID_ARG, "gguf_vision_weights: null argument");
    // siglip2.vision.* keys and defaults as src/siglip2_vision.cpp:27-34, 435-442
    const int64_t H = kv_int(g, "siglip2.vision.embedding_length", 1152);
    const int64_t F = kv_int(g, "siglip2.vision.feed_forward_length", 4304);
    const int64_t heads = kv_int(g, "siglip2.vision.attention.head_count", 16);
    const int64_t layers = kv_int(g, "siglip2.vision.block_count", 27);
    const int64_t patch = kv_int(g, "siglip2.vision.patch_size", 16);
    const int64_t n_patch = kv_int(g, "siglip2.vision.num_patches", 256);
    const int64_t chan = kv_int(g, "siglip2.vision.num_channels", 3);
    const double eps = kv_float(g, "siglip2.vision.layer_norm_eps", 1e-6);
    const int64_t side = (int64_t)std::llround(std::sqrt((double)n_patch));
    if (H <= 0 || H % 32 || F <= 0 || heads <= 0 || layers <= 0 || side * side != n_patch ||
        (patch * patch * chan) % 32)
        return fail(S2X_ERR_INVALID_ARG, "gguf: vision metadata out of range");
    const int64_t F_pad = ffn_down_kpad(g, "v", F);
    if (F_pad < F || F_pad - F >= 32 || F_pad % 32)
        return fail(S2X_ERR_UNSUPPORTED, "gguf: vision ffn_down K %lld for F %lld", (long long)F_pad,
                    (long long)F);
    s2x_vision_weights v{};
    v.hidden = (int32_t)H;
    v.inter = (int32_t)F;
    v.inter_pad = (int32_t)F_pad;
    v.n_head = (int32_t)heads;
    v.n_layer = (int32_t)layers;
    v.patch_dim = (int32_t)(patch * patch * chan);
    v.n_side = (int32_t)side;
    v.eps = (float)eps;
    int st;
    if ((st = bind_q8(g, "v.patch_embd.weight", v.patch_dim, v.patch_dim, H, &v.patch_w)) ||
        (st = bind_vec(g, "v.patch_embd.bias", H, &v.patch_b)) ||
        (st = bind_vec(g, "v.position_embd.weight", n_patch * H, &v.pos_embd)) ||
        (st = bind_vec(g, "v.post_ln.weight", H, &v.post_ln_w)) ||
        (st = bind_vec(g, "v.post_ln.bias", H, &v.post_ln_b)) ||
        (st = bind_vec(g, "v.head.probe", H, &v.probe)) ||
        (st = bind_q8(g, "v.head.attn_q.weight", H, H, H, &v.hq_w)) ||
        (st = bind_vec(g, "v.head.attn_q.bias", H, &v.hq_b)) ||
        (st = bind_q8(g, "v.head.attn_k.weight", H, H, H, &v.hk_w)) ||
        (st = bind_vec(g, "v.head.attn_k.bias", H, &v.hk_b)) ||
        (st = bind_q8(g, "v.head.attn_v.weight", H, H, H, &v.hv_w)) ||
        (st = bind_vec(g, "v.head.attn_v.bias", H, &v.hv_b)) ||
        (st = bind_q8(g, "v.head.attn_o.weight", H, H, H, &v.ho_w)) ||
        (st = bind_vec(g, "v.head.attn_o.bias", H, &v.ho_b)) ||
        (st = bind_vec(g, "v.head.ln.weight", H, &v.hln_w)) ||
        (st = bind_vec(g, "v.head.ln.bias", H, &v.hln_b)) ||
        (st = bind_q8(g, "v.head.ffn_up.weight", H, H, F, &v.hup_w)) ||
        (st = bind_vec(g, "v.head.ffn_up.bias", F, &v.hup_b)) ||
        (st = bind_vec(g, "v.head.ffn_down.bias", H, &v.hdown_b)) ||
        (st = bind_layers(g, "v", layers, H, F, F_pad, g->vision_layers, &v.down_f16)))
        return st;
    int head_f16 = 0;
    if ((st = bind_down(g, "v.head.ffn_down.weight", F, F_pad, H, &v.hdown_w, &head_f16)))
        return st;
    if (head_f16 != v.down_f16)
        return fail(S2X_ERR_UNSUPPORTED, "gguf: v.head.ffn_down type differs from the layers'");
    v.layers = g->vision_layers.data();
    *w = v;
    return S2X_OK;
}

int s2x_gguf_text_weights(s2x_gguf *g, s2x_text_weights *w) {
    if (!g || !w) return fail(S2X_ERR_INVALID_ARG, "gguf_text_weights: null argument");
    // siglip2.text.* keys and defaults as src/siglip2_text.cpp:27-34, 434-441
    const int64_t H = kv_int(g, "siglip2.text.embedding_length", 1152);
    const int64_t F = kv_int(g, "siglip2.text.feed_forward_length", 4304);
    const int64_t heads = kv_int(g, "siglip2.text.attention.head_count", 16);
    const int64_t layers = kv_int(g, "siglip2.text.block_count", 27);
    const int64_t vocab = kv_int(g, "siglip2.text.vocab_size", 256000);
    const int64_t max_pos = kv_int(g, "siglip2.text.max_position_embeddings", 64);
    const int64_t proj = kv_int(g, "siglip2.text.projection_size", H);
    const double eps = kv_float(g, "siglip2.text.layer_norm_eps", 1e-6);
    if (H <= 0 || H % 32 || F <= 0 || heads <= 0 || layers <= 0 || vocab <= 0 || max_pos <= 0 ||
        proj <= 0)
        return fail(S2X_ERR_INVALID_ARG, "gguf: text metadata out of range");
    const int64_t F_pad = ffn_down_kpad(g, "t", F);
    if (F_pad < F || F_pad - F >= 32 || F_pad % 32)
        return fail(S2X_ERR_UNSUPPORTED, "gguf: text ffn_down K %lld for F %lld", (long long)F_pad,
                    (long long)F);
    s2x_text_weights t{};
    t.hidden = (int32_t)H;
    t.inter = (int32_t)F;
    t.inter_pad = (int32_t)F_pad;
    t.n_head = (int32_t)heads;
    t.n_layer = (int32_t)layers;
    t.vocab = (int32_t)vocab;
    t.max_pos = (int32_t)max_pos;
    t.proj = (int32_t)proj;
    t.eps = (float)eps;
    int st;
    if ((st = bind_q8(g, "t.token_embd.weight", H, H, vocab, &t.tok_embd)) ||
        (st = bind_vec(g, "t.position_embd.weight", max_pos * H, &t.pos_embd)) ||
        (st = bind_vec(g, "t.final_ln.weight", H, &t.final_ln_w)) ||
        (st = bind_vec(g, "t.final_ln.bias", H, &t.final_ln_b)) ||
        (st = bind_q8(g, "t.head.weight", H, H, proj, &t.head_w)) ||
        (st = bind_vec(g, "t.head.bias", proj, &t.head_b)) ||
        (st = bind_layers(g, "t", layers, H, F, F_pad, g->text_layers, &t.down_f16)))
        return st;
    t.layers = g->text_layers.data();
    *w = t;
    return S2X_OK;
}

int s2x_gguf_score_params(s2x_gguf *g, float *logit_scale, float *logit_bias) {
    if (!g || !logit_scale || !logit_bias) return fail(S2X_ERR_INVALID_ARG, "gguf_score_params: null argument");
    // mm.logit_scale / mm.logit_bias: one F32 value each (src/siglip2_score.cpp:71-72)
    const float *s = nullptr, *b = nullptr;
    int st;
    if ((st = bind_vec(g, "mm.logit_scale", 1, &s)) || (st = bind_vec(g, "mm.logit_bias", 1, &b))) return st;
    *logit_scale = s[0];
    *logit_bias = b[0];
    return S2X_OK;
}

}  // extern "C"
