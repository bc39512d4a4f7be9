// s2x_mmq.hip -- Q8_0 (weights) x Q8_1 (activations) GEMM on gfx950 int8 MFMA.
//
// Y[m, n] = sum_kb  fmaf((float)I_kb[m,n], dw[n,kb] * dx[m,kb], acc)
//
// One v_mfma_i32_32x32x32_i8 consumes exactly one 32-value Q8 block, so its
// int32 result IS the per-block dot I_kb (exact).  The block's fp16 scales
// are widened to f32; their product is exact (11+11 significant bits), and
// the accumulation runs over kb in order with one fused multiply-add per
// block, the same arithmetic as the CPU restatement of ggml's scalar
// vec_dot_q8_0_q8_0 -- so results match it bit for bit.
//
// Tiling: a workgroup owns a BM x BN output tile (rows m = tokens, columns
// n = output features), split over WM x WN waves; a wave owns TM x TN
// 32x32 MFMA subtiles.  A stage of KS blocks of X (BM rows) and W (BN rows)
// is staged through LDS with a 16-byte row pad so the 16-byte operand reads
// of a wave (32 rows x 2 halves) fall into distinct banks.  Two LDS buffers:
// the next stage's global loads are in flight while the current one feeds
// the MFMAs.
//
// MFMA operand/result layout (32x32x32 i8): lane l supplies row (l & 31) of
// A (X) and column (l & 31) of B (W), 16 consecutive k-bytes at offset
// 16*(l >> 5) of the block -- the same k split for A and B, so the block dot
// is complete.  The result register r of lane l holds
//   row 8*(r/4) + 4*(l/32) + (r%4), column (l & 31).
#include "s2x_device.h"
#include "s2x_kernels.h"

namespace s2x {

template <int BM, int BN, int WM, int WN, int KS>
struct MmqCfg {
    static constexpr int NT = WM * WN * WAVE;        // threads
    static constexpr int TM = BM / WM / 32;          // subtiles per wave (rows)
    static constexpr int TN = BN / WN / 32;          // subtiles per wave (cols)
    static constexpr int ROWB = KS * QK + 16;        // LDS row pitch in bytes
    static constexpr int XCH = BM * KS * 2 / NT;     // 16-byte X chunks per thread
    static constexpr int WCH = BN * KS * 2 / NT;     // 16-byte W chunks per thread
    static constexpr int XSC = (BM * KS + NT - 1) / NT;  // X scales per thread
    static constexpr int WSC = (BN * KS + NT - 1) / NT;  // W scales per thread
    static constexpr int LDS_X = BM * ROWB;
    static constexpr int LDS_W = BN * ROWB;
    static constexpr int LDS_STAGE = LDS_X + LDS_W + (BM + BN) * KS * 4;
    static_assert(BM % (WM * 32) == 0 && BN % (WN * 32) == 0, "tile");
    static_assert((BM * KS * 2) % NT == 0 && (BN * KS * 2) % NT == 0, "chunks");
};

template <int BM, int BN, int WM, int WN, int KS, int EPI>
__global__ __launch_bounds__(WM *WN *WAVE) void k_mmq(
    const int8_t *__restrict__ xq, const uint32_t *__restrict__ xds,
    const int8_t *__restrict__ wq, const float *__restrict__ wd, int M, int N, int KB,
    float *__restrict__ y, int64_t ldy, EpiParams epi) {
    using C = MmqCfg<BM, BN, WM, WN, KS>;
    extern __shared__ __align__(16) uint8_t lds[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int m_tiles = (M + BM - 1) / BM, n_tiles = (N + BN - 1) / BN;
    int tmi, tni;
    tile_coords<8>(blockIdx.x, gridDim.x, m_tiles, n_tiles, tmi, tni);
    const int m0 = tmi * BM, n0 = tni * BN;
    const int64_t K_pad = (int64_t)KB * QK;

    int kb_begin = 0, kb_end = KB;
    if (EPI == EPI_DUMP_I) {
        kb_begin = (int)epi.dump_kb;
        kb_end = kb_begin + 1;
    }
    const int n_stages = (kb_end - kb_begin + KS - 1) / KS;

    v4i xr[C::XCH], wr[C::WCH];
    float xsr[C::XSC], wsr[C::WSC];

    auto gload = [&](int stage) {
        const int kb0 = kb_begin + stage * KS;
#pragma unroll
        for (int i = 0; i < C::XCH; ++i) {
            const int idx = tid + i * C::NT;
            const int r = idx / (KS * 2), c = idx % (KS * 2);
            const int m = m0 + r, kb = kb0 + (c >> 1);
            v4i v = {0, 0, 0, 0};
            if (m < M && kb < kb_end)
                v = *reinterpret_cast<const v4i *>(xq + (int64_t)m * K_pad + (int64_t)kb * QK + (c & 1) * 16);
            xr[i] = v;
        }
#pragma unroll
        for (int i = 0; i < C::WCH; ++i) {
            const int idx = tid + i * C::NT;
            const int r = idx / (KS * 2), c = idx % (KS * 2);
            const int n = n0 + r, kb = kb0 + (c >> 1);
            v4i v = {0, 0, 0, 0};
            if (n < N && kb < kb_end)
                v = *reinterpret_cast<const v4i *>(wq + (int64_t)n * K_pad + (int64_t)kb * QK + (c & 1) * 16);
            wr[i] = v;
        }
#pragma unroll
        for (int i = 0; i < C::XSC; ++i) {
            const int idx = tid + i * C::NT;  // idx = r * KS + k
            float v = 0.0f;
            if (idx < BM * KS) {
                const int r = idx / KS, k = idx % KS;
                const int m = m0 + r, kb = kb0 + k;
                if (EPI != EPI_DUMP_I && m < M && kb < kb_end)  // the dump reads no scales
                    v = f16_bits_to_f32((uint16_t)(xds[(int64_t)m * KB + kb] & 0xffffu));
            }
            xsr[i] = v;
        }
#pragma unroll
        for (int i = 0; i < C::WSC; ++i) {
            const int idx = tid + i * C::NT;
            float v = 0.0f;
            if (idx < BN * KS) {
                const int r = idx / KS, k = idx % KS;
                const int n = n0 + r, kb = kb0 + k;
                if (EPI != EPI_DUMP_I && n < N && kb < kb_end) v = wd[(int64_t)n * KB + kb];
            }
            wsr[i] = v;
        }
    };
    auto sstore = [&](int buf) {
        uint8_t *base = lds + buf * C::LDS_STAGE;
        uint8_t *xs = base;
        uint8_t *ws = base + C::LDS_X;
        float *xd = reinterpret_cast<float *>(base + C::LDS_X + C::LDS_W);  // [KS][BM]
        float *wdl = xd + KS * BM;                                          // [KS][BN]
#pragma unroll
        for (int i = 0; i < C::XCH; ++i) {
            const int idx = tid + i * C::NT;
            const int r = idx / (KS * 2), c = idx % (KS * 2);
            *reinterpret_cast<v4i *>(xs + r * C::ROWB + c * 16) = xr[i];
        }
#pragma unroll
        for (int i = 0; i < C::WCH; ++i) {
            const int idx = tid + i * C::NT;
            const int r = idx / (KS * 2), c = idx % (KS * 2);
            *reinterpret_cast<v4i *>(ws + r * C::ROWB + c * 16) = wr[i];
        }
#pragma unroll
        for (int i = 0; i < C::XSC; ++i) {
            const int idx = tid + i * C::NT;
            if (idx < BM * KS) xd[(idx % KS) * BM + idx / KS] = xsr[i];
        }
#pragma unroll
        for (int i = 0; i < C::WSC; ++i) {
            const int idx = tid + i * C::NT;
            if (idx < BN * KS) wdl[(idx % KS) * BN + idx / KS] = wsr[i];
        }
    };

    float acc[C::TM][C::TN][16];
#pragma unroll
    for (int a = 0; a < C::TM; ++a)
#pragma unroll
        for (int b = 0; b < C::TN; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;
    v16i dump[C::TM][C::TN];

    const int wrow0 = wm * (BM / WM);  // wave's first tile row
    const int wcol0 = wn * (BN / WN);
    const int lr = lane & 31;
    const int lh = lane >> 5;

    gload(0);
    sstore(0);
    __syncthreads();

    for (int s = 0; s < n_stages; ++s) {
        const int buf = s & 1;
        if (s + 1 < n_stages) gload(s + 1);

        const uint8_t *base = lds + buf * C::LDS_STAGE;
        const uint8_t *xs = base;
        const uint8_t *ws = base + C::LDS_X;
        const float *xd = reinterpret_cast<const float *>(base + C::LDS_X + C::LDS_W);
        const float *wdl = xd + KS * BM;
        const int kb0 = kb_begin + s * KS;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            if (kb0 + kk >= kb_end) break;
            v4i af[C::TM], bf[C::TN];
#pragma unroll
            for (int a = 0; a < C::TM; ++a)
                af[a] = *reinterpret_cast<const v4i *>(xs + (wrow0 + a * 32 + lr) * C::ROWB + kk * QK + lh * 16);
#pragma unroll
            for (int b = 0; b < C::TN; ++b)
                bf[b] = *reinterpret_cast<const v4i *>(ws + (wcol0 + b * 32 + lr) * C::ROWB + kk * QK + lh * 16);
            float dwv[C::TN];
#pragma unroll
            for (int b = 0; b < C::TN; ++b) dwv[b] = wdl[kk * BN + wcol0 + b * 32 + lr];
            float dxv[C::TM][16];
#pragma unroll
            for (int a = 0; a < C::TM; ++a)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const v4f t = *reinterpret_cast<const v4f *>(xd + kk * BM + wrow0 + a * 32 + 8 * g + 4 * lh);
                    dxv[a][4 * g + 0] = t.x;
                    dxv[a][4 * g + 1] = t.y;
                    dxv[a][4 * g + 2] = t.z;
                    dxv[a][4 * g + 3] = t.w;
                }
#pragma unroll
            for (int a = 0; a < C::TM; ++a)
#pragma unroll
                for (int b = 0; b < C::TN; ++b) {
                    const v16i zero = {};
                    const v16i I = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[a], bf[b], zero, 0, 0, 0);
                    if (EPI == EPI_DUMP_I) {
                        dump[a][b] = I;
                    } else {
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            acc[a][b][r] = fmaf((float)I[r], dwv[b] * dxv[a][r], acc[a][b][r]);
                    }
                }
        }

        if (s + 1 < n_stages) sstore(buf ^ 1);
        __syncthreads();
    }

    // epilogue
#pragma unroll
    for (int a = 0; a < C::TM; ++a)
#pragma unroll
        for (int b = 0; b < C::TN; ++b) {
            const int n = n0 + wcol0 + b * 32 + lr;
            if (n >= N) continue;
            float bias = 0.0f;
            if (EPI == EPI_BIAS || EPI == EPI_BIAS_GELU || EPI == EPI_BIAS_RESID) bias = epi.bias[n];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wrow0 + a * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (m >= M) continue;
                if (EPI == EPI_DUMP_I) {
                    reinterpret_cast<int32_t *>(y)[(int64_t)m * ldy + n] = dump[a][b][r];
                    continue;
                }
                float v = acc[a][b][r];
                if (EPI == EPI_BIAS) {
                    v = v + bias;
                } else if (EPI == EPI_BIAS_GELU) {
                    v = gelu_tanh(v + bias);
                } else if (EPI == EPI_BIAS_RESID) {
                    const int64_t rm = epi.resid_rows > 0 ? (int64_t)m % epi.resid_rows : (int64_t)m;
                    v = (v + bias) + epi.resid[rm * epi.ld_resid + n];
                }
                y[(int64_t)m * ldy + n] = v;
            }
        }
}

template <int BM, int BN, int WM, int WN, int KS, int EPI>
static hipError_t run_mmq(const WeightView &w, const int8_t *xq, const uint32_t *xds,
                          int64_t M, float *y, int64_t ldy, const EpiParams &epi,
                          hipStream_t stream) {
    using C = MmqCfg<BM, BN, WM, WN, KS>;
    const int m_tiles = (int)((M + BM - 1) / BM), n_tiles = (int)((w.N + BN - 1) / BN);
    const int G = m_tiles * n_tiles;
    const size_t lds = 2 * (size_t)C::LDS_STAGE;
    auto kern = k_mmq<BM, BN, WM, WN, KS, EPI>;
    static bool attr_set = false;  // idempotent; a racing second call repeats it harmlessly
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL(kern, dim3(G), dim3(C::NT), lds, stream, xq, xds, w.qs, w.d, (int)M,
                       (int)w.N, (int)(w.K_pad / QK), y, ldy, epi);
    return hipGetLastError();
}

hipError_t launch_mmq(const WeightView &w, const int8_t *xq, const uint32_t *xds, int64_t M,
                      float *y, int64_t ldy, const EpiParams &epi, hipStream_t stream) {
    if (M == 0 || w.N == 0) return hipSuccess;
    constexpr int BM = 128, BN = 128, WM = 2, WN = 2, KS = 4;
    switch (epi.kind) {
    case EPI_NONE: return run_mmq<BM, BN, WM, WN, KS, EPI_NONE>(w, xq, xds, M, y, ldy, epi, stream);
    case EPI_BIAS: return run_mmq<BM, BN, WM, WN, KS, EPI_BIAS>(w, xq, xds, M, y, ldy, epi, stream);
    case EPI_BIAS_GELU:
        return run_mmq<BM, BN, WM, WN, KS, EPI_BIAS_GELU>(w, xq, xds, M, y, ldy, epi, stream);
    case EPI_BIAS_RESID:
        return run_mmq<BM, BN, WM, WN, KS, EPI_BIAS_RESID>(w, xq, xds, M, y, ldy, epi, stream);
    case EPI_DUMP_I:
        return run_mmq<BM, BN, WM, WN, KS, EPI_DUMP_I>(w, xq, xds, M, y, ldy, epi, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace s2x
