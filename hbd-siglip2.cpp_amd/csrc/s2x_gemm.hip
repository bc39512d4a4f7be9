// s2x_gemm.hip -- Q8_0 (weights) x Q8_1 (activations) GEMM on gfx950 int8
// MFMA, with the fused epilogues of the SigLIP2 encoder block.
//
//   Y[m, n] = epilogue( sum over K blocks kb, in block order:
//                         acc = fmaf((float)I_kb[m,n], dw[n,kb] * dx[m,kb], acc) )
//
// I_kb is the exact int32 dot of the 32 quants of block kb; dw and dx are the
// fp16 block scales (src/cuda/siglip2_custom_mmq.cu:259-267 is the same
// per-block rescale).  The K loop carries acc' = acc * 2^-26 (below); per
// 32 x 32 output subtile and K block:
//   * I'  = I * 2^-26: one v_mfma_i32_32x32x32_i8 (exact) accumulating onto
//           the bits of the float c0 = 0x3E22F983 (1/2pi, an inline
//           constant: no registers), so that the result read as a float is
//           c0 + I * 2^-26 exactly (|I| <= 2^19 stays inside c0's binade),
//           then one v_mfma_f32_32x32x8_f16 adding -c0 as three exact f16
//           products (every partial sum is a multiple of 2^-26 below 1/4:
//           exact in any order);
//   * s   = dx[i] * dw[j] as one v_mfma_f32_32x32x8_f16 whose A holds dx in
//           k-slot 0 and B holds dw in k-slot 0, every other slot zero: each
//           output is one exact f16 x f16 product in f32;
//   * acc' = fmaf(I', s, acc') on the VALU.
// The scaling commutes with every rounding: all terms are multiples of
// 2^-74 (f16 scales are multiples of 2^-24) and |acc| < 2^19 * 65504^2 *
// KB < 2^80, so acc' never reaches the subnormals nor acc overflow, and
// fmaf(I', s, acc') = 2^-26 fmaf(I, s, acc) at every step; the epilogue
// multiplies by 2^26 (exact).  The outputs are those of the per-block fma
// chain bit for bit.
// Three MFMAs (96 matrix-pipe cycles) against 16 VALU instructions (64
// cycles): the matrix pipe bounds this formulation at a third of the int8
// MFMA peak.
//
// Work decomposition.  128 x 128 output tiles, one per workgroup of 8 waves
// (each 32 x 64: 2 subtiles), two workgroups per CU so that one's epilogue
// and pipeline fill overlap the other's K loop.  GEMMs of too few such tiles
// to give every CU two (batch 1, M = 729) run 64 x 128 tiles of 4 waves
// whose K stages are scheduled for a lone wave's latency instead.  The K
// loop runs over stages of KS blocks whose operands (X and W quants and
// scales) arrive by LDS DMA (buffer_load ... lds) into a ring of NS stage
// buffers, NS - 1 stages ahead (NS = 2; 3 or 4 in the latency form); one
// workgroup barrier per stage.
//
// Scale layouts: X scales are the Q8_1 ds words of the activation
// (ds[m * ld_ds + kb] = fp16 d | fp16 s << 16, the block_q8_1 scale pair);
// W scales are fp16 bits transposed, dT[kb * ldT + n].
//
// LDS layout of one stage (bytes):
//   XQ  [KS][128 rows][32]  X quants, the two 16-byte chunks of row r at
//                            chunk position c ^ swz(r)
//   WQ  [KS][128 rows][32]  W quants, same swizzle
//   XS  [128][KS] u32        X ds words, a row's KS blocks together (as in
//                            the ds plane: one 16-byte DMA lane per row)
//   WS  [KS][128] u16        W scales in the dT plane's column order
//                            (columns j and j + 32 of each 64-column half
//                            in one 32-bit word)
// A fragment read (lane l: row l & 31, chunk l >> 5, 16 bytes) then touches
// 16 distinct 16-byte bank groups per 16 lanes: no bank conflicts.
#include "s2x_device.h"
#include "s2x_kernels.h"

#include <type_traits>
#include <utility>

namespace s2x {
namespace gemm {

constexpr int BN = 128;  // output tile columns
constexpr int GM = 8;    // tile-row group of the tile order
constexpr int RM_N_TILES = 12;  // at most this many column tiles: row-major tile order
constexpr int BUF_DW3 = 0x00020000;  // buffer resource word 3: raw 32-bit dwords

// BM x 128 tiles (BM 128, 64 or 32), waves of 32 TM x 32 TN outputs (BM /
// 32 TM along M, 128 / 32 TN along N); stages of KS K blocks in a ring of NS stage buffers
// (NS - 1 stages in flight).  Throughput form (LAT false): as many
// workgroups per CU as two rings allow, each K block its own scheduling
// region, <= 128 VGPRs (4 waves per SIMD cover each other's latency).
// Latency form (LAT true, for GEMMs of too few tiles to give a SIMD more
// than one or two waves): a stage's KS blocks are one scheduling region --
// all their fragments read up front, their MFMAs interleaved -- with up to
// 256 VGPRs, so that a lone wave keeps its matrix pipe busy.
template <int KS_, int NS_, int BM_ = 128, bool LAT_ = false, int TM_ = 1, int TN_ = 2>
struct Cfg {
    static constexpr int TM = TM_, TN = TN_, BM = BM_, KS = KS_, NS = NS_;
    static constexpr bool LAT = LAT_;
    // waves of 32 TM x 32 TN outputs, WN of them along N
    static constexpr int WN = BN / (32 * TN), NWAVE = BM / (32 * TM) * WN, NT = NWAVE * WAVE;
    static constexpr int XQ = 0;                  // [KS][BM][32] X quants
    static constexpr int WQ = XQ + KS * BM * 32;  // [KS][BN][32] W quants
    // [XS_ROWS][KS] u32 X ds words: at least 64 rows, the rows one X-scale
    // DMA instruction writes (rows past a 32-row tile are never read)
    static constexpr int XS_ROWS = BM < 64 ? 64 : BM;
    static constexpr int XS = WQ + KS * BN * 32;
    static constexpr int WS = XS + KS * XS_ROWS * 4;  // [KS][BN] fp16 W scales
    static constexpr int STAGE = WS + KS * BN * 2;
    static constexpr int LDS_BYTES = NS * STAGE;
    static constexpr int WG_PER_CU = 2 * LDS_BYTES <= 163840 ? 2 : 1;
    static constexpr int WPE = LAT ? 2 : WG_PER_CU * NWAVE / 4;  // waves per SIMD
    // DMA instructions per stage: QPX X-quant and QPW W-quant per wave (each
    // 32 rows of one block: KS BM / 32 and 4 KS per stage); the scales, 16
    // bytes per lane (a row's 4 consecutive ds words, or 8 W scales of one
    // block), by the first NSX + 1 waves: waves 0 .. NSX - 1 the X scales
    // of 64 rows each, wave NSX the W scales.  The issue cost of these
    // instructions, not their bytes, is what the K loop feels, hence the
    // scales in as few of them as their 16-byte rows allow.
    static constexpr int NSX = BM < 64 ? 1 : BM / 64;
    static constexpr int QPX = KS * (BM / 32) / NWAVE, QPW = KS * (BN / 32) / NWAVE;
    static_assert(KS == 4, "stage of 4 blocks: one 16-byte ds row per X row");
    static_assert(BM == 128 || BM == 64 || (BM == 32 && LAT && TN == 1), "tile rows");
    static_assert(QPX >= 1 && QPW >= 1 && QPX <= KS && QPW <= KS, "DMA split");
    static_assert(NS == 2 || (LAT && NS <= 4), "ring: two stages, or up to four in the latency form");
    static_assert(NSX + 1 <= NWAVE, "scale DMA waves");
    static_assert(LDS_BYTES * WG_PER_CU <= 163840, "LDS");
    static_assert(NWAVE * 5120 <= LDS_BYTES, "epilogue scratch");
};

typedef __attribute__((address_space(3))) void lds_void;

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>), in order
template <class F, int... J>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, J...>) {
    (f(std::integral_constant<int, J>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// chunk permutation of the two 16-byte chunks of a 32-byte row
__device__ __forceinline__ int swz(int r) { return ((r >> 2) ^ (r >> 3)) & 1; }

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                      uint8_t *lds_wave_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds_wave_base, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint8_t *lds_wave_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds_wave_base, 4, voff, 0, 0, 0);
}
// A per-lane offset past every buffer's range (num_records <= 2^31 - 1):
// that lane's DMA returns zeros and reads no memory.
constexpr uint32_t OOB_OFF = 0x80000000u;

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ int clip32(int64_t bytes) {
    return (int)(bytes < 0 ? 0 : bytes > 0x7fffffff ? 0x7fffffff : bytes);
}

// Output tile of logical index T: groups of GM row tiles walk N together;
// where N has few tiles (N = 1,152: 9), row-major, so the workgroups that
// share a row tile's X panel (every column tile of it) are dispatched side
// by side and stream its K blocks through the L2 together (batch-32
// out-projection and fc2: 31 % and 15 % fewer bytes fetched, same time).
__device__ __forceinline__ void tile_of(int T, int m_tiles, int n_tiles, int &tm, int &tn) {
    if (n_tiles <= RM_N_TILES) {
        tm = T / n_tiles;
        tn = T - tm * n_tiles;
        return;
    }
    const int group_size = GM * n_tiles;
    const int group = T / group_size;
    const int first_m = group * GM;
    const int gm = min(GM, m_tiles - first_m);
    const int in_group = T - group * group_size;
    tm = first_m + in_group % gm;
    tn = in_group / gm;
}

// One K block's MFMA operands for a wave's TM x 2 subtiles.  The scale
// operands are the 4-half (two-dword) f16 vectors of a 32x32x8 MFMA: dword 0
// holds the scale in its low half (k slot 0 on lanes 0..31), every other
// half is zero, and lanes 32..63 (k slots 4..7) are zero in both operands,
// so no product is 0 x inf.
template <int TM, int TN>
struct Frag {
    v4i a[TM], b[TN];
    uint32_t xw[TM], wp;  // the raw ds words and W-scale word (operands built at use)
};

// Epilogue of one wave's 32 TM x 32 TN block (rows mw.., columns nw..), from
// the accumulators in registers; wscr: 5,120 bytes of LDS of this wave.
// The GELU -> Q8_1 / f16 and QKV epilogues take 32 x 64 blocks (TN = 2).
// The product is acc * scale (a power of two: exact), so that mm + bias is
// one fmaf(acc, scale, bias), the same bits as (acc * scale) + bias.
constexpr int EPI_SCRATCH = 5120;
template <int TM, int TN, int EPI>
__device__ __forceinline__ void epilogue(float (&acc)[TM][TN][16], float scale, const float (&bias_v)[TN], int lane,
                                         int mw, int nw, int M, int N, float *__restrict__ y,
                                         int64_t ldy, const EpiParams &epi, uint8_t *wscr) {
    static_assert(TN == 2 || EPI == EPI_NONE || EPI == EPI_BIAS || EPI == EPI_BIAS_GELU ||
                      EPI == EPI_BIAS_RESID || EPI == EPI_DUMP_I,
                  "32 x 32 waves take the plain epilogues only");
    const int lr = lane & 31, lh = lane >> 5;
    if constexpr (EPI == EPI_GELU_Q81) {
        // GELU(mm + bias), then Q8_1 exactly as k_quantize_q8_1 over
        // rows of q_kpad values (columns >= N are zeros): each 32 x 32
        // subtile is one quant block per row; it goes through LDS so that
        // lane pairs own a row (16 values each).  Columns >= N need no
        // branch: their W quants arrive as zeros (rows past N) and their
        // W scales are the zeroed padding of the dT plane, so acc is +0,
        // the bias 0, and GELU(+0) = +0.
        constexpr int P = 36;  // floats per scratch row
        float *scr = reinterpret_cast<float *>(wscr);
        const int row = lane >> 1, half = lane & 1;
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int nb0 = nw + b * 32;  // first column of this quant block
                if (nb0 >= epi.q_kpad) continue;  // wave-uniform
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    scr[(8 * (r >> 2) + 4 * lh + (r & 3)) * P + lr] =
                        gelu_tanh(fmaf(acc[a][b][r], scale, bias_v[b]));
                float v[16];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const v4f t = *reinterpret_cast<const v4f *>(scr + row * P + half * 16 + 4 * j);
                    v[4 * j] = t[0]; v[4 * j + 1] = t[1]; v[4 * j + 2] = t[2]; v[4 * j + 3] = t[3];
                }
                float am = 0.0f;
#pragma unroll
                for (int j = 0; j < 16; ++j) am = fmaxf(am, fabsf(v[j]));
                am = fmaxf(am, dpp_f<0xb1>(am));  // partner lane (xor 1)
                const float d = am / 127.0f;
                const float inv = am != 0.0f ? 127.0f / am : 0.0f;
                int qi[16], qs = 0;
                if (q8_any_sat(inv)) {
#pragma unroll
                    for (int j = 0; j < 16; ++j) qi[j] = q8_round(v[j], inv);
                } else {
#pragma unroll
                    for (int j = 0; j < 16; ++j) qi[j] = q8_round_fast(v[j], inv);
                }
#pragma unroll
                for (int j = 0; j < 16; ++j) qs += qi[j];
                qs += dpp_i<0xb1>(qs);
                const int m = mw + a * 32 + row;
                if (m < M) {
                    const int64_t off = (int64_t)m * epi.q_kpad + nb0 + half * 16;
                    *reinterpret_cast<uint4 *>(epi.q_out8 + off) =
                        make_uint4(pack4_i8(qi[0], qi[1], qi[2], qi[3]), pack4_i8(qi[4], qi[5], qi[6], qi[7]),
                                   pack4_i8(qi[8], qi[9], qi[10], qi[11]),
                                   pack4_i8(qi[12], qi[13], qi[14], qi[15]));
                    if (half == 0)
                        epi.q_ds[(int64_t)m * epi.q_ldds + nb0 / QK] =
                            (uint32_t)f32_to_f16_bits(d) |
                            ((uint32_t)f32_to_f16_bits((float)qs * d) << 16);
                }
            }
    } else if constexpr (EPI == EPI_GELU_F16) {
        // GELU(mm + bias) rounded to f16, rows of h_kpad halves (columns
        // N .. h_kpad - 1 zero): the f16 activation of an F16 weight
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int n = nw + b * 32 + lr;
                if (n >= epi.h_kpad) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = mw + a * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                    if (m < M)
                        epi.h_out[(int64_t)m * epi.h_ld + n] =
                            n < N ? f32_to_f16(gelu_tanh(fmaf(acc[a][b][r], scale, bias_v[b]))) : (_Float16)0.0f;
                }
            }
    } else if constexpr (EPI == EPI_QKV) {
        // (mm + bias) in f32, then f16, into Q / K [seg][head][pos][d_pad]
        // or V^T [seg][head][dv_pad][pos]; padding slots are not written
        const int H = epi.n_head * epi.d_head;
        const float inv_dh = 1.0f / (float)epi.d_head;
        if (H % 64 == 0 && nw < 2 * H && epi.d_head % 8 == 0 && epi.d_pad % 8 == 0) {
            // a Q or K tile: each 32-row half of the wave's 32 x 64 block
            // goes through LDS so that each 8-column chunk of a row (8
            // consecutive d of one head) leaves as one 16-byte store
            constexpr int P = 72;  // halves per scratch row
            _Float16 *scr = reinterpret_cast<_Float16 *>(wscr);
            _Float16 *dst0 = nw < H ? epi.q : epi.k;
            const int hd0 = nw < H ? 0 : H;
#pragma unroll
            for (int a = 0; a < TM; ++a) {
                int rmv[4];  // row map entries, loaded before the stores
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    rmv[i] = epi.rowmap[min(mw + a * 32 + ((lane + 64 * i) >> 3), M - 1)];
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        scr[(8 * (r >> 2) + 4 * lh + (r & 3)) * P + b * 32 + lr] =
                            f32_to_f16(fmaf(acc[a][b][r], scale, bias_v[b]));
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int id = lane + 64 * i, row = id >> 3, c = (id & 7) * 8;
                    const int m = mw + a * 32 + row, n = nw + c;
                    if (m >= M || n >= N) continue;
                    const int rm = rmv[i];
                    if (rm == ROW_NONE) continue;
                    const int hd = n - hd0;
                    const int h = small_div(hd, epi.d_head, inv_dh), d = hd - h * epi.d_head;
                    const int64_t sh = (int64_t)(rm >> 16) * epi.n_head + h;
                    const v8h v = *reinterpret_cast<const v8h *>(scr + row * P + c);
                    *reinterpret_cast<v8h *>(dst0 + (sh * epi.len_pad + (rm & 0xffff)) * epi.d_pad + d) = v;
                }
            }
        } else if (H % 64 == 0 && nw >= 2 * H) {
            // a V tile: V^T rows are positions, so each 32-row half goes
            // through LDS transposed (column-major, rows shifted by the
            // first position's offset within its 8-position chunk) and
            // each lane writes one column -- one d of one head: up to 32
            // consecutive positions -- as 16-byte stores where the
            // destination is 16-byte aligned, 2-byte stores at the ends
            constexpr int PT = 40;  // halves per scratch column (shift <= 7, 32 rows)
            _Float16 *scr = reinterpret_cast<_Float16 *>(wscr);
            const int n = nw + lane;
            const int hd = n - 2 * H, h = small_div(max(hd, 0), epi.d_head, inv_dh);
            const int d = hd - h * epi.d_head;
#pragma unroll
            for (int a = 0; a < TM; ++a) {
                const int mr = mw + a * 32;
                const int rows = min(32, M - mr);  // wave-uniform, may be <= 0
                int rm_first = 0, rm_last = 0;
                if (rows > 0) {
                    rm_first = epi.rowmap[mr];
                    rm_last = epi.rowmap[mr + rows - 1];
                }
                // one segment, consecutive positions: the common case (the
                // rows between two covered rows of one segment are covered)
                const bool run = rows > 0 && rm_first != ROW_NONE && rm_last != ROW_NONE &&
                                 (rm_last >> 16) == (rm_first >> 16) &&
                                 (rm_last & 0xffff) - (rm_first & 0xffff) == rows - 1;
                const int shift = run ? (rm_first & 0xffff) & 7 : 0;
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            scr[(b * 32 + lr) * PT + shift + 8 * q + 4 * lh + j] =
                                f32_to_f16(fmaf(acc[a][b][4 * q + j], scale, bias_v[b]));
                if (rows > 0 && n < N) {
                    const _Float16 *col = scr + lane * PT;
                    if (run) {
                        const int64_t sh = (int64_t)(rm_first >> 16) * epi.n_head + h;
                        _Float16 *dst =
                            epi.vt + (sh * epi.dv_pad + d) * epi.len_pad + (rm_first & 0xffff) - shift;
                        // positions [shift, shift + rows) of the 8-aligned window dst[0 ..)
                        const int lo = shift, hi = shift + rows;
                        const int a0 = (lo + 7) & ~7, a1 = hi & ~7;
                        if (a0 <= a1) {
                            for (int i = lo; i < a0; ++i) dst[i] = col[i];
                            for (int i = a0; i < a1; i += 8)
                                *reinterpret_cast<v8h *>(dst + i) = *reinterpret_cast<const v8h *>(col + i);
                            for (int i = a1; i < hi; ++i) dst[i] = col[i];
                        } else {
                            for (int i = lo; i < hi; ++i) dst[i] = col[i];
                        }
                    } else {
                        for (int i = 0; i < rows; ++i) {
                            const int rm = epi.rowmap[mr + i];
                            if (rm == ROW_NONE) continue;
                            const int64_t sh = (int64_t)(rm >> 16) * epi.n_head + h;
                            epi.vt[(sh * epi.dv_pad + d) * epi.len_pad + (rm & 0xffff)] = col[i];
                        }
                    }
                }
            }
        } else {
            // any H: one 2-byte store per element
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int n = nw + b * 32 + lr;
                if (n >= N) continue;
                const int part = small_div(n, H, 1.0f / (float)H), hd = n - part * H;
                const int h = small_div(hd, epi.d_head, inv_dh), d = hd - h * epi.d_head;
                _Float16 *dst = part == 0 ? epi.q : part == 1 ? epi.k : epi.vt;
#pragma unroll
                for (int a = 0; a < TM; ++a)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int m = mw + a * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                        if (m >= M) continue;
                        const int rm = epi.rowmap[m];
                        if (rm == ROW_NONE) continue;
                        const int64_t sh = (int64_t)(rm >> 16) * epi.n_head + h;
                        const int pos = rm & 0xffff;
                        const int64_t off = part < 2 ? (sh * epi.len_pad + pos) * epi.d_pad + d
                                                     : (sh * epi.dv_pad + d) * epi.len_pad + pos;
                        dst[off] = f32_to_f16(fmaf(acc[a][b][r], scale, bias_v[b]));
                    }
            }
        }
    } else {
        // (mm + bias) [GELU | + residual], through buffer loads and stores
        // whose bounds drop the rows past M (and the columns past N, sent
        // out of range): no branch per element.  Each 32-row half's
        // residual loads are all issued before its first store (y may be
        // the residual itself: each element is read, then written, by
        // one lane).
        constexpr uint32_t OOB = 0x80000000u;
        const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(y + (int64_t)mw * ldy), (short)0, clip32((int64_t)(M - mw) * ldy * 4), BUF_DW3);
        const bool rmod = epi.resid_rows > 0;
        const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(epi.resid + (rmod ? 0 : (int64_t)mw * epi.ld_resid)), (short)0,
            EPI == EPI_BIAS_RESID
                ? clip32((rmod ? epi.resid_rows : (int64_t)(M - mw)) * epi.ld_resid * 4)
                : 0,
            BUF_DW3);
        // Every row of the wave's block inside M and a plain residual (not
        // the position rows): the lane's first row and its column in the
        // vector offset (out of range past N), the row steps 8 (r >> 2) +
        // (r & 3) as scalar offsets -- no address arithmetic per element.
        // Rows past M stay with the form below, whose vector offsets alone
        // carry every row.
        if (mw + 32 * TM <= M && !rmod && EPI != EPI_DUMP_I && EPI != EPI_BIAS_GELU) {
            const uint32_t sy = (uint32_t)ldy * 4u, sr = (uint32_t)epi.ld_resid * 4u;
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b) {
                    const int n = nw + b * 32 + lr;
                    const int r0 = a * 32 + 4 * lh;
                    const uint32_t vy = n < N ? (uint32_t)(r0 * (int)ldy + n) * 4u : OOB;
                    float res[16];
                    if constexpr (EPI == EPI_BIAS_RESID) {
                        const uint32_t vr = n < N ? (uint32_t)(r0 * (int)epi.ld_resid + n) * 4u : OOB;
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const uint32_t dm = (uint32_t)(8 * (r >> 2) + (r & 3));
                            res[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rr, vr, dm * sr, 0));
                        }
                    }
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        float v = acc[a][b][r];
                        if (EPI == EPI_NONE) {
                            v = v * scale;
                        } else if (EPI == EPI_BIAS) {
                            v = fmaf(v, scale, bias_v[b]);
                        } else if (EPI == EPI_BIAS_RESID) {
                            v = fmaf(v, scale, bias_v[b]) + res[r];
                        }
                        const uint32_t dm = (uint32_t)(8 * (r >> 2) + (r & 3));
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), yr, vy, dm * sy, 0);
                    }
                }
            return;
        }
#pragma unroll
        for (int a = 0; a < TM; ++a) {
            float res[TN][16];
            if constexpr (EPI == EPI_BIAS_RESID) {
                // residual row of this lane's first row in the half; the
                // others are at most 27 rows further (one wrap when
                // resid_rows >= 28)
                const int R = (int)epi.resid_rows;
                const int m_first = mw + a * 32 + 4 * lh;
                const int r_first = rmod ? m_first % R : m_first - mw;
#pragma unroll
                for (int b = 0; b < TN; ++b) {
                    const int n = nw + b * 32 + lr;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int dm = 8 * (r >> 2) + (r & 3);
                        int rm = r_first + dm;
                        if (rmod) rm = R >= 28 ? (rm >= R ? rm - R : rm) : rm % R;
                        const uint32_t off =
                            n < N ? (uint32_t)(rm * (int)epi.ld_resid + n) * 4u : OOB;
                        const uint32_t bits = __builtin_amdgcn_raw_buffer_load_b32(rr, off, 0, 0);
                        res[b][r] = __builtin_bit_cast(float, bits);
                    }
                }
            }
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                const int n = nw + b * 32 + lr;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float v = acc[a][b][r];  // EPI_DUMP_I: the raw bits
                    if (EPI == EPI_NONE) {
                        v = v * scale;
                    } else if (EPI == EPI_BIAS) {
                        v = fmaf(v, scale, bias_v[b]);
                    } else if (EPI == EPI_BIAS_GELU) {
                        v = gelu_tanh(fmaf(v, scale, bias_v[b]));
                    } else if (EPI == EPI_BIAS_RESID) {
                        v = fmaf(v, scale, bias_v[b]) + res[b][r];
                    }
                    const int mr = a * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                    const uint32_t off = n < N ? (uint32_t)(mr * (int)ldy + n) * 4u : OOB;
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), yr,
                                                          off, 0, 0);
                }
            }
        }
    }
}

template <class C, int EPI>
__global__ __launch_bounds__(C::NT) __attribute__((amdgpu_waves_per_eu(C::WPE))) void k_gemm(
    const uint8_t *__restrict__ xq, const uint32_t *__restrict__ xds, int64_t ld_ds,
    const uint8_t *__restrict__ wq, const uint16_t *__restrict__ wdT, int64_t ldT, int M, int N,
    int KB, float *__restrict__ y, int64_t ldy, EpiParams epi) {
    constexpr int BM = C::BM, NS = C::NS, KS = C::KS, STAGE = C::STAGE, TM = C::TM;
    constexpr int XQ = C::XQ, WQ = C::WQ, XS = C::XS, WS = C::WS;
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    constexpr int TN = C::TN;
    const int wm = wave / C::WN, wn = wave % C::WN;
    const int lr = lane & 31, lh = lane >> 5;
    const int m_tiles = (M + BM - 1) / BM, n_tiles = (N + BN - 1) / BN;
    int tm, tn;
    tile_of(xcd_linear(blockIdx.x, gridDim.x), m_tiles, n_tiles, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int KB_all = KB;
    const int64_t row_bytes = (int64_t)KB_all * QK;  // X and W rows: all KB blocks
    // a K split: this workgroup's blocks kbs .. kbs + KB - 1 (EPI_NONE)
    int kbs = 0;
    if (EPI == EPI_NONE && epi.kb_split > 0) {
        kbs = (int)blockIdx.y * epi.kb_split;
        KB = min(epi.kb_split, KB - kbs);
        y += (int64_t)blockIdx.y * epi.y_split;
    }
    const int n_st = (KB + KS - 1) / KS;

    // Per-lane DMA source offsets (relative to the tile's first row / column;
    // the K position goes into the scalar offset).
    //   X quants, instructions t < QPX: i = QPX wave + t, block i % KS, rows
    //             32 (i / KS) .. + 31 (= 32 (QPX wave / KS) for every t)
    //   W quants, instructions t < QPW: likewise with QPW
    //   X scales: waves w < NSX, rows 64 w + lane, the ds words of blocks
    //             k0 .. k0 + 3 (16 bytes)
    //   W scales: wave NSX, block lane / 16, columns 8 (lane % 16) .. + 7
    uint32_t vqx, vqw, vxs, vws;
    {
        const int rx = 32 * (C::QPX * wave / KS) + (lane >> 1);
        vqx = (uint32_t)(rx * row_bytes) + (uint32_t)(((lane & 1) ^ swz(rx)) * 16);
        const int rw = 32 * (C::QPW * wave / KS) + (lane >> 1);
        vqw = (uint32_t)(rw * row_bytes) + (uint32_t)(((lane & 1) ^ swz(rw)) * 16);
        vxs = (uint32_t)((min(wave, C::NSX - 1) * 64 + lane) * ld_ds * 4);
        vws = (uint32_t)((lane >> 4) * ldT * 2 + (lane & 15) * 16);
    }
    // (the bases start at block kbs; the ranges end where the planes end)
    const __amdgpu_buffer_rsrc_t xr_live = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(xq + (int64_t)m0 * row_bytes + kbs * QK), (short)0,
        clip32((int64_t)(M - m0) * row_bytes - kbs * QK), BUF_DW3);
    const __amdgpu_buffer_rsrc_t wr_live = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(wq + (int64_t)n0 * row_bytes + kbs * QK), (short)0,
        clip32((int64_t)(N - n0) * row_bytes - kbs * QK), BUF_DW3);
    const __amdgpu_buffer_rsrc_t xsr_live = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(xds + (int64_t)m0 * ld_ds + kbs), (short)0,
        clip32((int64_t)(M - m0) * ld_ds * 4 - kbs * 4), BUF_DW3);
    const __amdgpu_buffer_rsrc_t wsr_live = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(wdT + (int64_t)kbs * ldT + n0), (short)0,
        clip32(((int64_t)(KB_all - kbs) * ldT - n0) * 2), BUF_DW3);
    const __amdgpu_buffer_rsrc_t none = __builtin_amdgcn_make_buffer_rsrc((void *)xq, (short)0, 0, BUF_DW3);

    // Issue the DMA of stage g into buffer g % NS.  Rows past M or N return
    // zeros through the per-lane offset (the vector offset alone exceeds the
    // range), and a stage past the last is issued through zero-size buffers
    // (no memory is read).  No read goes past block KB - 1, whatever the
    // range check does with the scalar offset: a partial last stage (KB %
    // KS blocks, KB >= KS) is fetched as the window of the last KS blocks,
    // kpos(g) = KB - KS, so its block kb0 + j lands in slot j + shift of the
    // stage buffer (shift = kb0 - kpos); a GEMM of fewer than KS blocks has
    // one partial stage, fetched by the first issue (outside the K loop)
    // with a zero-size buffer per missing block and out-of-range lanes for
    // the missing scales.  ROLE (a constant per wave: 1 X scales, 2 W
    // scales, 0 neither) is a template value, so that no branch splits the
    // K loop.
    // PART: 0 the X quants, 1 the W quants, 2 the scales, -1 all three
    auto kpos = [&](int g) { return KB >= KS ? min(g * KS, KB - KS) : g * KS; };
    auto issue = [&](int g, auto role, auto part, auto first) {
        constexpr int ROLE = decltype(role)::value, PART = decltype(part)::value;
        const bool live = g < n_st;
        uint8_t *sb = lds + (g % NS) * STAGE;
        if constexpr (decltype(first)::value) {
            if (KB < KS) {
                // the only stage, blocks 0 .. KB - 1 of KS
#pragma unroll
                for (int t = 0; t < C::QPX; ++t) {
                    const int i = C::QPX * wave + t, j = i % KS;
                    dma16(j < KB ? xr_live : none, vqx, j * 32, sb + XQ + j * BM * 32 + (i / KS) * 1024);
                }
#pragma unroll
                for (int t = 0; t < C::QPW; ++t) {
                    const int i = C::QPW * wave + t, j = i % KS;
                    dma16(j < KB ? wr_live : none, vqw, j * 32, sb + WQ + j * BN * 32 + (i / KS) * 1024);
                }
                if constexpr (ROLE == 1) {
                    // one 4-byte DMA per ds word: 16 rows x KS words per
                    // instruction, the words of missing blocks out of range
#pragma unroll
                    for (int t = 0; t < 64 / 16; ++t) {
                        const int row = 64 * wave + 16 * t + (lane >> 2), w = lane & 3;
                        const uint32_t off = w < KB ? (uint32_t)((row * ld_ds + w) * 4) : OOB_OFF;
                        dma4(xsr_live, off, sb + XS + (64 * wave + 16 * t) * 16);
                    }
                } else if constexpr (ROLE == 2) {
                    dma16(wsr_live, (lane >> 4) < KB ? vws : OOB_OFF, 0, sb + WS);  // lane: block lane / 16
                }
                return;
            }
        }
        const __amdgpu_buffer_rsrc_t xr = live ? xr_live : none, wr = live ? wr_live : none;
        const __amdgpu_buffer_rsrc_t xsr = live ? xsr_live : none, wsr = live ? wsr_live : none;
        const uint32_t k0 = (uint32_t)kpos(g);
        if constexpr (PART == 0 || PART < 0) {
#pragma unroll
            for (int t = 0; t < C::QPX; ++t) {
                const int i = C::QPX * wave + t, j = i % KS;
                dma16(xr, vqx, (k0 + j) * 32, sb + XQ + j * BM * 32 + (i / KS) * 1024);
            }
        }
        if constexpr (PART == 1 || PART < 0) {
#pragma unroll
            for (int t = 0; t < C::QPW; ++t) {
                const int i = C::QPW * wave + t, j = i % KS;
                dma16(wr, vqw, (k0 + j) * 32, sb + WQ + j * BN * 32 + (i / KS) * 1024);
            }
        }
        if constexpr (PART == 2 || PART < 0) {
            if constexpr (ROLE == 1)
                dma16(xsr, vxs, k0 * 4, sb + XS + wave * 64 * 16);
            else if constexpr (ROLE == 2)
                dma16(wsr, vws, (uint32_t)(k0 * ldT * 2), sb + WS);
        }
    };
    using All = std::integral_constant<int, -1>;

    // Stage g + 1 visible to every wave: this wave's DMA of it has landed,
    // then the barrier.  After it no wave reads stage g's buffer any more, so
    // the DMA of stage g + 2 may refill it.
    auto arrive = [&]() {
        wait_vm<0>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };

    // fragment addresses (bytes within a stage buffer) of this lane
    const int xrow = wm * 32 * TM + lr, wcol = wn * 32 * TN + lr;
    const int a_off = XQ + xrow * 32 + ((lh ^ swz(lr)) * 16);
    const int b_off = WQ + wcol * 32 + ((lh ^ swz(lr)) * 16);
    const int sx_off = XS + xrow * 16;
    // the 32-bit word of W scales (column j | column j + 32 << 16 of a
    // 64-column group) holding this lane's columns, and the low half of the
    // X ds word (the scale d), both masked to zero on lanes 32..63 (k slots
    // 4..7); a 32 x 32 wave takes the half of the word its columns are
    const int sw_off = WS + (wn * TN / 2) * 128 + lr * 4;
    const int sw_sh = TN == 1 ? 16 * (wn & 1) : 0;
    const uint32_t xmask = lh ? 0u : 0xffffu, wmask = lh ? 0u : ~0u;
    // slot j of the stage buffer (a constant in the K loop; the last
    // stage's block j + its window shift)
    auto load_frag = [&](const uint8_t *sb, int j, Frag<TM, TN> &f) {
#pragma unroll
        for (int a = 0; a < TM; ++a)
            f.a[a] = *reinterpret_cast<const v4i *>(sb + a_off + j * BM * 32 + a * 32 * 32);
#pragma unroll
        for (int b = 0; b < TN; ++b)
            f.b[b] = *reinterpret_cast<const v4i *>(sb + b_off + j * BN * 32 + b * 32 * 32);
#pragma unroll
        for (int a = 0; a < TM; ++a) f.xw[a] = *reinterpret_cast<const uint32_t *>(sb + sx_off + j * 4 + a * 32 * 16);
        f.wp = *reinterpret_cast<const uint32_t *>(sb + sw_off + j * BN * 2);
    };
    // the scale operands of subtile (a, b), from the raw words: the VALU
    // work sits with the MFMAs that use it, not with the (early) reads
    auto sx_op = [&](const Frag<TM, TN> &f, int a) { return v2i{(int)(f.xw[a] & xmask), 0}; };
    auto sw_op = [&](const Frag<TM, TN> &f, int b) {
        const uint32_t w = f.wp & wmask;
        return v2i{(int)(TN == 2 ? (b ? w >> 16 : w & 0xffffu) : (w >> sw_sh) & 0xffffu), 0};
    };

    float acc[TM][TN][16];
    Frag<TM, TN> F;

    // One K block, subtile k = 2a + b, in three MFMAs and 16 fmas:
    //   D = X.W^T + 0x3E22F983 (int8 MFMA whose accumulator starts at the
    //       bits of c0 = 1/2pi, an inline constant, whose ulp is 2^-26: D
    //       read as a float is c0 + I 2^-26 exactly, |I| <= 32 * 128 * 128
    //       = 2^19 and c0's mantissa 0x22F983 +- 2^19 stays in [0, 2^23));
    //   I' = D - c0 (an f16 MFMA adding -0.125 x 1, -1119/256 x 2^-7 and
    //       -387/8192 x 2^-13 from k-slots 0..2 to the accumulator D: exact,
    //       so I' is I_kb * 2^-26);
    //   s = dx[i] * dw[j] (the scale tile);
    //   acc' = fmaf(I', s, acc') on the VALU.
    // The matrix pipe (3 x 32 cycles) rather than the VALU (16 x 4 cycles)
    // bounds a subtile-block; the convert-on-VALU form it replaces needed 32
    // VALU instructions (128 cycles).  Results are consumed right away (no
    // slot ring inside the wave, which keeps the kernel at <= 128 VGPRs and
    // 4 waves per SIMD): the SIMD's other waves cover the MFMA latency.
    constexpr int NSUB = TM * TN;
    // f16 (-0.125, -1119/256, -387/8192, 0) x (1, 2^-7, 2^-13, 0) in k-slots
    // 0..3, lanes 32..63 (slots 4..7) zero: the products sum to -c0
    const v2i cA = {lh ? 0 : (int)0xC45FB000u, lh ? 0 : 0xAA0C};
    const v2i cB = {lh ? 0 : 0x20003C00, lh ? 0 : 0x0800};
    // hook(): called once the block's last block dot is issued (where the
    // throughput form reads the next block's fragments)
    auto compute = [&](const Frag<TM, TN> &f, int kb, auto &&hook) {
        const v16f zf = {};
        const v16i zi = {};
        // c0's bits in every element (the latency form's splat; the
        // throughput form names the inline constant itself, below)
        const v16i magic = 0x3E22F983;
        if constexpr (EPI == EPI_DUMP_I) {
#pragma unroll
            for (int k = 0; k < NSUB; ++k) {
                const int a = k / TN, b = k % TN;
                const v16i D = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[a], f.b[b], zi, 0, 0, 0);
                if (k == NSUB - 1) hook();
                if (kb == (int)epi.dump_kb) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        // through a scalar: bit_cast of a vector element
                        // operand compiles to element 0 here
                        const int t = D[r];
                        acc[a][b][r] = __builtin_bit_cast(float, t);
                    }
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < NSUB; ++k) {
                const int a = k / TN, b = k % TN;
                v16i D;
                if constexpr (!C::LAT) {
                    // The accumulator operand as the inline constant 1/2pi
                    // (0x3E22F983) in the instruction: LLVM folds the splat
                    // only where one MFMA uses it, and otherwise keeps it in
                    // 16 VGPRs that every block dot reads -- at <= 128 VGPRs
                    // for 4 waves per SIMD.  Written this way the K loop
                    // takes ~100 VGPRs.  The one reader of D is the
                    // conversion MFMA right below, with D exactly as its
                    // accumulator operand: the dependency the compiler
                    // itself schedules back to back with no wait states
                    // (an MFMA whose srcC exactly overlaps the previous
                    // MFMA's result); no VALU instruction reads D.
                    asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, 0.15915494"
                                 : "=&v"(D) : "v"(f.a[a]), "v"(f.b[b]));
                } else {
                    D = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[a], f.b[b], magic, 0, 0, 0);
                }
                if (k == NSUB - 1) hook();
                const v16f I = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, cA),
                                                                    __builtin_bit_cast(v4h, cB),
                                                                    __builtin_bit_cast(v16f, D), 0, 0, 0);
                const v16f S = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, sx_op(f, a)),
                                                                    __builtin_bit_cast(v4h, sw_op(f, b)), zf, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[a][b][r] = fmaf(I[r], S[r], acc[a][b][r]);
            }
        }
        // throughput form: one scheduling region per block, nothing moves
        // across blocks
        if constexpr (!C::LAT) __builtin_amdgcn_sched_barrier(0);
    };

    float bias_v[TN];
#pragma unroll
    for (int b = 0; b < TN; ++b) {
        const int n = n0 + wcol + b * 32;
        bias_v[b] = EPI != EPI_NONE && EPI != EPI_DUMP_I && n < N ? epi.bias[n] : 0.0f;
    }
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

    // Latency form, software-pipelined over K blocks (each output's fma
    // chain is the only serial dependency; a block's MFMAs depend on
    // nothing of the block before).  Slot j of a stage: read block j + 1's
    // fragments, issue block j's MFMAs (block dots, scale tiles, then the
    // conversions, into ring entry j % 2) and run block j - 1's fmas from
    // ring entry (j - 1) % 2, one MFMA per five VALU instructions, so that
    // the wave's matrix pipe and VALU work side by side.  Block 3's fmas
    // run in slot 0 of the next stage (after its barrier); the fmas stay in
    // block order.
    struct Ring {
        v16f I[NSUB], S[NSUB];
    };
    auto mfma_group = [&](const Frag<TM, TN> &f, Ring &R) {
        v16i D[NSUB];
        const v16f zf = {};
        const v16i magic = 0x3E22F983;
#pragma unroll
        for (int k = 0; k < NSUB; ++k)
            D[k] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[k / TN], f.b[k % TN], magic, 0, 0, 0);
#pragma unroll
        for (int k = 0; k < NSUB; ++k)
            R.S[k] = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, sx_op(f, k / TN)),
                                                          __builtin_bit_cast(v4h, sw_op(f, k % TN)), zf, 0, 0, 0);
#pragma unroll
        for (int k = 0; k < NSUB; ++k)
            R.I[k] = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, cA), __builtin_bit_cast(v4h, cB),
                                                          __builtin_bit_cast(v16f, D[k]), 0, 0, 0);
    };
    auto fma_group = [&](const Ring &R) {
#pragma unroll
        for (int k = 0; k < NSUB; ++k)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                acc[k / TN][k % TN][r] = fmaf(R.I[k][r], R.S[k][r], acc[k / TN][k % TN][r]);
    };
    // the slot's order: fragment reads first, then MFMA / VALU alternating
    auto slot_order = [&]() {
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
        for (int i = 0; i < 3 * NSUB; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
        }
    };
    // NS - 1 stages in flight: the DMA instructions this wave issues per
    // stage (a constant of its role), so that the wait for a stage lets
    // the younger stages' instructions stay outstanding (loads complete in
    // order)
    auto k_loop_pipelined = [&](auto role) {
        constexpr int ROLE = decltype(role)::value;
        constexpr int DPS = C::QPX + C::QPW + (ROLE != 0 ? 1 : 0);
        issue(0, role, All{}, std::true_type{});
        static_for<NS - 1>([&](auto sc) { issue(1 + decltype(sc)::value, role, All{}, std::false_type{}); });
        wait_vm<(NS - 1) * DPS>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        // ring entry 1 starts at zero: the first stage's slot 0 runs its
        // fmas as fmaf(0, 0, acc) = acc (acc is never -0)
        Ring R[2];
#pragma unroll
        for (int k = 0; k < NSUB; ++k) R[1].I[k] = R[1].S[k] = v16f{};
        Frag<TM, TN> Fs[2];
        // every stage but the last: KS blocks, no branch
        for (int g = 0; g < n_st - 1; ++g) {
            const uint8_t *sb = lds + (g % NS) * STAGE;
            load_frag(sb, 0, Fs[0]);
            static_for<KS>([&](auto jc) {
                constexpr int j = decltype(jc)::value;
                if constexpr (j + 1 < KS) load_frag(sb, j + 1, Fs[(j + 1) & 1]);
                mfma_group(Fs[j & 1], R[j & 1]);
                fma_group(R[(j + 1) & 1]);  // block j - 1 (slot 0: the previous stage's block 3)
                slot_order();
                __builtin_amdgcn_sched_barrier(0);
            });
            // stage g + 1 landed (stages g + 2 .. g + NS - 1 may still be
            // in flight), every wave past stage g: its buffer takes stage
            // g + NS
            wait_vm<(NS - 2) * DPS>();
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            issue(g + NS, role, All{}, std::false_type{});
        }
        // the last stage: the previous stage's block 3, then nb = 1 .. KS
        // blocks one at a time, block kb0 + j in slot j + shift (a partial
        // stage was fetched as the window of the last KS blocks)
        fma_group(R[1]);
        const uint8_t *sb = lds + ((n_st - 1) % NS) * STAGE;
        const int kb0 = (n_st - 1) * KS, nb = KB - kb0, shift = kb0 - kpos(n_st - 1);
        static_for<KS>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            if (j < nb) {
                load_frag(sb, j + shift, Fs[0]);
                mfma_group(Fs[0], R[0]);
                fma_group(R[0]);
            }
        });
    };

    auto k_loop = [&](auto role) {
    if constexpr (C::LAT && EPI != EPI_DUMP_I) {
        k_loop_pipelined(role);
        return;
    }
    issue(0, role, All{}, std::true_type{});
    arrive();  // the first stage visible
    if constexpr (C::LAT) issue(1, role, All{}, std::false_type{});
    // stage g computed while stage g + 1 loads; each block's fragments are
    // read right before its MFMAs (the other waves of the SIMD cover the
    // LDS latency)
    for (int g = 0; g < n_st - 1; ++g) {
        const uint8_t *sb = lds + (g % NS) * STAGE;
        const int kb0 = g * KS;
        if constexpr (C::LAT) {
            // every fragment of the stage first, then its blocks in order
            Frag<TM, TN> Fs[KS];
            static_for<KS>([&](auto jc) { load_frag(sb, decltype(jc)::value, Fs[decltype(jc)::value]); });
            static_for<KS>([&](auto jc) { compute(Fs[decltype(jc)::value], kb0 + decltype(jc)::value, [] {}); });
        } else {
            // the next stage's DMA in three parts after blocks 0, 1 and 2:
            // spread over the stage rather than in one burst after the
            // barrier, when every wave of the CU starts reading fragments.
            // Block j + 1's fragments are read once block j's last block
            // dot is issued (into the registers of the other fragment set:
            // the K loop has the VGPRs since the block dots' accumulator
            // operand is an inline constant).
            Frag<TM, TN> Fp[2];
            load_frag(sb, 0, Fp[0]);
            static_for<KS>([&](auto jc) {
                constexpr int j = decltype(jc)::value;
                compute(Fp[j & 1], kb0 + j, [&] {
                    if constexpr (j + 1 < KS) load_frag(sb, j + 1, Fp[(j + 1) & 1]);
                });
                if constexpr (j < 3) issue(g + 1, role, std::integral_constant<int, j>{}, std::false_type{});
            });
        }
        arrive();
        // the latency form's MFMAs may sink below the barrier (its stage is
        // one scheduling region): its next DMA goes out after the barrier,
        // a whole stage before the wait for it
        if constexpr (C::LAT) issue(g + 2, role, All{}, std::false_type{});
    }
    {
        // the last stage: nb = 1 .. KS blocks, block kb0 + j in slot
        // j + shift (a partial stage was fetched as the last KS blocks)
        const uint8_t *sb = lds + ((n_st - 1) % NS) * STAGE;
        const int kb0 = (n_st - 1) * KS, nb = KB - kb0, shift = kb0 - kpos(n_st - 1);
        static_for<KS>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            if (j < nb) {
                load_frag(sb, j + shift, F);
                compute(F, kb0 + j, [] {});
            }
        });
    }
    };
    if (wave < C::NSX)
        k_loop(std::integral_constant<int, 1>{});
    else if (wave == C::NSX)
        k_loop(std::integral_constant<int, 2>{});
    else
        k_loop(std::integral_constant<int, 0>{});

    // ----------------------------------------------------------------------
    // Epilogue.  The LDS is free scratch once the last (empty) stage's DMA
    // has landed and every wave has read its last fragments.
    // ----------------------------------------------------------------------
    if constexpr (EPI == EPI_GELU_Q81 || EPI == EPI_QKV) {
        wait_vm<0>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    // acc = acc' * 2^26 (exact), folded into the epilogue's first operation
    epilogue<TM, TN, EPI>(acc, 67108864.0f, bias_v, lane, m0 + wm * 32 * TM, n0 + wn * 32 * TN, M, N, y, ldy, epi,
                      lds + wave * EPI_SCRATCH);
    // Every DMA this wave issued has landed before the workgroup ends.
    wait_vm<0>();
}

template <class C, int EPI>
hipError_t run(const WeightView &w, const int8_t *xq, const uint32_t *xds, int64_t ld_ds,
               int64_t M, float *y, int64_t ldy, const EpiParams &epi, hipStream_t stream) {
    auto kern = k_gemm<C, EPI>;
    static bool attr_set = false;  // idempotent; a racing second call repeats it harmlessly
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 C::LDS_BYTES);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const int64_t tiles = ((M + C::BM - 1) / C::BM) * ((w.N + BN - 1) / BN);
    const int64_t KB = w.K_pad / QK;
    const unsigned splits = epi.kb_split > 0 ? (unsigned)((KB + epi.kb_split - 1) / epi.kb_split) : 1u;
    // without scales (the block-dot dump) the scale DMA reads a zero-size
    // buffer at a valid address
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles, splits), dim3(C::NT), C::LDS_BYTES, stream,
                       reinterpret_cast<const uint8_t *>(xq),
                       xds ? xds : reinterpret_cast<const uint32_t *>(xq), xds ? ld_ds : 0,
                       reinterpret_cast<const uint8_t *>(w.qs), w.dT, w.ldT, (int)M, (int)w.N,
                       (int)(w.K_pad / QK), y, ldy, epi);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// F16 weight x f16 activation, f32 accumulation (GGML_OP_MUL_MAT with an
// F16 weight, as the reference's converter stores ffn_down: K = 4304 is
// not a multiple of 32).  Same tiles, waves, tile order and LDS-DMA ring as
// k_gemm; a K block is 32 halves (64-byte rows, four 16-byte chunks, chunk
// c of row r at position c ^ ((r >> 2) & 3)), two v_mfma_f32_32x32x16_f16
// per subtile accumulate straight into the outputs: no scales, no VALU.
// ---------------------------------------------------------------------------
struct CfgH {
    static constexpr int BM = 128, KS = 2, NS = 2, NWAVE = 8, NT = NWAVE * WAVE;
    static constexpr int XQ = 0, WQ = XQ + KS * BM * 64, STAGE = WQ + KS * BN * 64;
    static constexpr int LDS_BYTES = NS * STAGE;  // 64 KiB: two workgroups per CU
    static constexpr int DMA_N = 2 * (KS * BM / 16) / NWAVE;  // 16 rows of a block per instruction
    static_assert(NWAVE * EPI_SCRATCH <= LDS_BYTES, "epilogue scratch");
};

__device__ __forceinline__ int swz4(int r) { return (r >> 2) & 3; }

template <int EPI>
__global__ __launch_bounds__(CfgH::NT) __attribute__((amdgpu_waves_per_eu(4))) void k_gemm_f16(
    const uint8_t *__restrict__ xh, const uint8_t *__restrict__ wh, int M, int N, int KB,
    float *__restrict__ y, int64_t ldy, EpiParams epi) {
    using C = CfgH;
    constexpr int BM = C::BM, KS = C::KS, STAGE = C::STAGE, XQ = C::XQ, WQ = C::WQ;
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lh = lane >> 5;
    const int m_tiles = (M + BM - 1) / BM, n_tiles = (N + BN - 1) / BN;
    int tm, tn;
    tile_of(xcd_linear(blockIdx.x, gridDim.x), m_tiles, n_tiles, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int n_st = (KB + KS - 1) / KS;
    const int64_t row_bytes = (int64_t)KB * 64;

    // DMA: a stage is KS blocks x 128 rows of X and of W, 16 rows of one
    // block per instruction (lane: row lane / 4, chunk position lane % 4);
    // waves 0-3 fetch X, 4-7 W, instruction t of wave w: block t % KS, rows
    // 16 (G (w % 4) + t / KS) .. + 15, G = DMA_N / KS row groups per wave
    const int kind = wave >> 2;
    const __amdgpu_buffer_rsrc_t src_live = kind == 0
        ? __builtin_amdgcn_make_buffer_rsrc((void *)(xh + (int64_t)m0 * row_bytes), (short)0,
                                            clip32((int64_t)(M - m0) * row_bytes), BUF_DW3)
        : __builtin_amdgcn_make_buffer_rsrc((void *)(wh + (int64_t)n0 * row_bytes), (short)0,
                                            clip32((int64_t)(N - n0) * row_bytes), BUF_DW3);
    const __amdgpu_buffer_rsrc_t none = __builtin_amdgcn_make_buffer_rsrc((void *)xh, (short)0, 0, BUF_DW3);
    uint32_t voff[C::DMA_N];
#pragma unroll
    for (int t = 0; t < C::DMA_N; ++t) {
        const int r = 16 * (C::DMA_N / KS * (wave & 3) + t / KS) + (lane >> 2);
        voff[t] = (uint32_t)(r * row_bytes) + (uint32_t)(((lane & 3) ^ swz4(r)) * 16);
    }
    // blocks past KB (an odd KB's last stage, every block of a stage past
    // the last) through the zero-size buffer: nothing past the planes is
    // addressed
    auto issue = [&](int g) {
        uint8_t *sb = lds + (g & 1) * STAGE + (kind == 0 ? XQ : WQ);
        const uint32_t k0 = (uint32_t)(g * KS);
#pragma unroll
        for (int t = 0; t < C::DMA_N; ++t) {
            const int j = t % KS, grp = C::DMA_N / KS * (wave & 3) + t / KS;
            dma16((int)k0 + j < KB ? src_live : none, voff[t], (k0 + j) * 64,
                  sb + j * BM * 64 + grp * 1024);
        }
    };
    auto arrive = [&](int g) {
        wait_vm<0>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        issue(g + 1);
    };

    const int xrow = wm * 32 + lr;
    int a_off[2], b_off[2][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        a_off[h] = XQ + xrow * 64 + (((2 * h + lh) ^ swz4(xrow)) * 16);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int wc = wn * 64 + b * 32 + lr;
            b_off[b][h] = WQ + wc * 64 + (((2 * h + lh) ^ swz4(wc)) * 16);
        }
    }
    v16f acc_v[2] = {};
    auto block = [&](const uint8_t *sb, int j) {
        v8h a[2], bq[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            a[h] = *reinterpret_cast<const v8h *>(sb + a_off[h] + j * BM * 64);
#pragma unroll
            for (int b = 0; b < 2; ++b)
                bq[b][h] = *reinterpret_cast<const v8h *>(sb + b_off[b][h] + j * BN * 64);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int b = 0; b < 2; ++b)
                acc_v[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[h], bq[b][h], acc_v[b], 0, 0, 0);
    };

    issue(0);
    arrive(0);
    for (int g = 0; g < n_st - 1; ++g) {
        const uint8_t *sb = lds + (g & 1) * STAGE;
#pragma unroll
        for (int j = 0; j < KS; ++j) block(sb, j);
        arrive(g + 1);
    }
    {
        const uint8_t *sb = lds + ((n_st - 1) & 1) * STAGE;
        const int nb = KB - (n_st - 1) * KS;
#pragma unroll
        for (int j = 0; j < KS; ++j)
            if (j < nb) block(sb, j);
    }

    float acc[1][2][16];
    float bias_v[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int n = n0 + wn * 64 + b * 32 + lr;
        bias_v[b] = EPI != EPI_NONE && n < N ? epi.bias[n] : 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[0][b][r] = acc_v[b][r];
    }
    epilogue<1, 2, EPI>(acc, 1.0f, bias_v, lane, m0 + wm * 32, n0 + wn * 64, M, N, y, ldy, epi,
                     lds + wave * EPI_SCRATCH);
    wait_vm<0>();
}

template <int EPI>
hipError_t run_f16(const _Float16 *w16, int64_t K_pad, int64_t N, const _Float16 *x16, int64_t M,
                   float *y, int64_t ldy, const EpiParams &epi, hipStream_t stream) {
    auto kern = k_gemm_f16<EPI>;
    static bool attr_set = false;
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 CfgH::LDS_BYTES);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const int64_t tiles = ((M + CfgH::BM - 1) / CfgH::BM) * ((N + BN - 1) / BN);
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(CfgH::NT), CfgH::LDS_BYTES, stream,
                       reinterpret_cast<const uint8_t *>(x16), reinterpret_cast<const uint8_t *>(w16),
                       (int)M, (int)N, (int)(K_pad / QK), y, ldy, epi);
    return hipGetLastError();
}

}  // namespace gemm

// y = ((p_0 + p_1) + ...) [+ bias] [+ resid], 4 columns per thread (N % 4
// == 0) or 1; y may be resid itself (each element read, then written, by
// one thread)
template <bool VEC>
__global__ __launch_bounds__(256) void k_split_sum(const float *__restrict__ part, int n_split,
                                                   int64_t plane, int64_t M, int64_t N,
                                                   const float *__restrict__ bias,
                                                   const float *resid, int64_t ld_resid,
                                                   float *y, int64_t ldy) {
    constexpr int W = VEC ? 4 : 1;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t nq = N / W;
    if (i >= M * nq) return;
    const int64_t m = i / nq, n = (i - m * nq) * W;
    float v[W];
#pragma unroll
    for (int j = 0; j < W; ++j) v[j] = part[m * N + n + j];
    for (int s = 1; s < n_split; ++s)
#pragma unroll
        for (int j = 0; j < W; ++j) v[j] = v[j] + part[s * plane + m * N + n + j];
#pragma unroll
    for (int j = 0; j < W; ++j) {
        if (bias) v[j] = v[j] + bias[n + j];
        if (resid) v[j] = v[j] + resid[m * ld_resid + n + j];
    }
#pragma unroll
    for (int j = 0; j < W; ++j) y[m * ldy + n + j] = v[j];
}

hipError_t launch_gemm_split_k(const WeightView &w, const int8_t *xq, const uint32_t *xds,
                               int64_t ld_ds, int64_t M, float *y, int64_t ldy,
                               const EpiParams &epi, int n_split, float *part,
                               hipStream_t stream) {
    if (M == 0 || w.N == 0) return hipSuccess;
    const int64_t KB = w.K_pad / QK;
    const bool resid = epi.kind == EPI_BIAS_RESID;
    if ((epi.kind != EPI_NONE && !resid) || n_split < 1 || !part || ldy < w.N ||
        (resid && (!epi.resid || epi.ld_resid < w.N || epi.resid_rows != 0)))
        return hipErrorInvalidValue;
    // whole 4-block stages per range
    const int64_t per = ((KB + n_split - 1) / n_split + 3) / 4 * 4;
    const int64_t splits = (KB + per - 1) / per;
    EpiParams e{};
    e.kind = EPI_NONE;
    e.kb_split = (int)per;
    e.y_split = M * w.N;
    hipError_t err = launch_gemm(w, xq, xds, ld_ds, M, part, w.N, e, stream);
    if (err != hipSuccess) return err;
    const bool vec = w.N % 4 == 0 && ldy % 4 == 0 && (!resid || epi.ld_resid % 4 == 0);
    const int64_t n = M * (vec ? w.N / 4 : w.N);
    const unsigned grid = (unsigned)((n + 255) / 256);
    if (vec)
        hipLaunchKernelGGL(k_split_sum<true>, dim3(grid), dim3(256), 0, stream, part,
                           (int)splits, M * w.N, M, w.N, resid ? epi.bias : nullptr, resid ? epi.resid : nullptr,
                           epi.ld_resid, y, ldy);
    else
        hipLaunchKernelGGL(k_split_sum<false>, dim3(grid), dim3(256), 0, stream, part,
                           (int)splits, M * w.N, M, w.N, resid ? epi.bias : nullptr, resid ? epi.resid : nullptr,
                           epi.ld_resid, y, ldy);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// GEMMs of at most 8 rows (the pooling head's one query per image at batch
// 1, the text head's prompts).  The MFMA forms give each 32 x 32 output
// block one wave that walks the whole K chain (the head's fc2 at M = 1: 36
// waves for 135 blocks each), so such a GEMM takes the chain's latency on a
// few CUs.  Here a workgroup owns CW columns of every row: its threads first
// compute the int32 block dots of all (column, block) pairs at once -- v_dot4
// over int8, exact, each W block read once for every row -- into LDS, then
// one thread per output runs acc = fmaf((float)I_kb, dx_kb * dw_kb, acc) over
// the blocks in order.  That is the MFMA forms' chain (whose 2^-26 scaling
// is exact), so the bits are theirs.  CW = 8 columns (plain, bias, GELU and
// residual epilogues: the head's N = 1,152 GEMMs in 144 workgroups), or 32
// where the epilogue quantizes 32-column blocks (GELU -> Q8_1).
// ---------------------------------------------------------------------------
constexpr int GV_MAX_M = 8;
constexpr int GV_NT = 256;
constexpr int GV_IT = 8;    // (column, block) pairs per thread: CW KB <= 2,048
constexpr int GV_XIT = 12;  // 16-byte X chunks per thread: M K_pad <= 49,152
constexpr int GV_LDS_MAX = 96 * 1024;

// position of column n's scale in a dT row (WeightView: columns c + j and
// c + 32 + j of each 64-column group share a 32-bit word)
__device__ __forceinline__ int gv_dw_pos(int n) { return (n & ~63) | ((n & 31) << 1) | ((n >> 5) & 1); }

template <int CW>
static int64_t gv_lds_bytes(int64_t M, int64_t K_pad) {
    const int64_t KB = K_pad / QK;
    return M * K_pad + 4 * (M * KB + CW * KB + M * CW * KB + M * 32);
}

template <int CW, int EPI>
__global__ __launch_bounds__(GV_NT) void k_gemv(const int8_t *__restrict__ xq,
                                                const uint32_t *__restrict__ xds, int64_t ld_ds,
                                                const int8_t *__restrict__ wq,
                                                const uint16_t *__restrict__ wdT, int64_t ldT,
                                                int K_pad, int M, int N, float *__restrict__ y,
                                                int64_t ldy, EpiParams epi) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int KB = K_pad / QK, tid = threadIdx.x, n0 = blockIdx.x * CW;
    int8_t *xs = reinterpret_cast<int8_t *>(lds);                    // [M][K_pad]
    float *dxs = reinterpret_cast<float *>(lds + (int64_t)M * K_pad);  // [M][KB]
    float *dws = dxs + M * KB;                                         // [CW][KB], 0 past N
    float *ib = dws + CW * KB;                                         // [M][CW][KB]
    float *vr = ib + M * CW * KB;                                      // [M][32] (GELU -> Q8_1)

    // every load issued before the first is awaited: the W blocks of this
    // thread's pairs (pair i: column i / KB, block i % KB), the X chunks
    // and both planes of scales
    int4 wv[GV_IT][2];
#pragma unroll
    for (int j = 0; j < GV_IT; ++j) {
        const int i = tid + j * GV_NT, c = i / KB, kb = i - c * KB;
        wv[j][0] = wv[j][1] = int4{0, 0, 0, 0};
        if (i < CW * KB && n0 + c < N) {
            const int4 *p = reinterpret_cast<const int4 *>(wq + (int64_t)(n0 + c) * K_pad + kb * QK);
            wv[j][0] = p[0];
            wv[j][1] = p[1];
        }
    }
    // (unconditional loads of clamped indices, so that none waits behind a
    // branch: X rows of K_pad bytes back to back, the X ds words of pair i
    // = (row i / KB, block i % KB), the W scale of pair i)
    const int xch = M * (K_pad / 16);
    int4 xv[GV_XIT];
#pragma unroll
    for (int j = 0; j < GV_XIT; ++j)
        xv[j] = reinterpret_cast<const int4 *>(xq)[min(tid + j * GV_NT, xch - 1)];
    uint32_t dxv[GV_IT];
    uint16_t dwv[GV_IT];
#pragma unroll
    for (int j = 0; j < GV_IT; ++j) {
        const int i = tid + j * GV_NT;
        const int ix = min(i, M * KB - 1), iw = min(i, CW * KB - 1);
        dxv[j] = xds[(int64_t)(ix / KB) * ld_ds + ix % KB];
        dwv[j] = wdT[(int64_t)(iw % KB) * ldT + gv_dw_pos(min(n0 + iw / KB, N - 1))];
    }
    // (the stores as unconditional: a thread past the end rewrites the last
    // element with the value it already holds -- no branch for the loads to
    // sink into)
#pragma unroll
    for (int j = 0; j < GV_XIT; ++j) reinterpret_cast<int4 *>(xs)[min(tid + j * GV_NT, xch - 1)] = xv[j];
#pragma unroll
    for (int j = 0; j < GV_IT; ++j) {
        const int i = tid + j * GV_NT;
        const int ix = min(i, M * KB - 1), iw = min(i, CW * KB - 1);
        dxs[ix] = f16_bits_to_f32((uint16_t)(dxv[j] & 0xffffu));
        dws[iw] = n0 + iw / KB < N ? f16_bits_to_f32(dwv[j]) : 0.0f;
    }
    __syncthreads();

    // the block dots, each W block against every row
#pragma unroll
    for (int j = 0; j < GV_IT; ++j) {
        const int i = tid + j * GV_NT;
        const int c = i / KB, kb = i - c * KB;
        for (int m = 0; m < (i < CW * KB ? M : 0); ++m) {
            const int4 *xp = reinterpret_cast<const int4 *>(xs + (int64_t)m * K_pad + kb * QK);
            const int4 x0 = xp[0], x1 = xp[1];
            int d = __builtin_amdgcn_sdot4(x0.x, wv[j][0].x, 0, false);
            d = __builtin_amdgcn_sdot4(x0.y, wv[j][0].y, d, false);
            d = __builtin_amdgcn_sdot4(x0.z, wv[j][0].z, d, false);
            d = __builtin_amdgcn_sdot4(x0.w, wv[j][0].w, d, false);
            d = __builtin_amdgcn_sdot4(x1.x, wv[j][1].x, d, false);
            d = __builtin_amdgcn_sdot4(x1.y, wv[j][1].y, d, false);
            d = __builtin_amdgcn_sdot4(x1.z, wv[j][1].z, d, false);
            d = __builtin_amdgcn_sdot4(x1.w, wv[j][1].w, d, false);
            ib[(m * CW + c) * KB + kb] = (float)d;  // |d| <= 2^19: exact
        }
    }
    __syncthreads();

    // the chains: output (m, c) for thread m CW + c
    const int m = tid / CW, c = tid % CW, n = n0 + c;
    if (m < M) {
        const float *ip = ib + (m * CW + c) * KB, *xp = dxs + m * KB, *wp = dws + c * KB;
        float acc = 0.0f;
        for (int kb = 0; kb < KB; ++kb) acc = fmaf(ip[kb], xp[kb] * wp[kb], acc);  // dx dw: exact
        const bool live = n < N;
        const float bias = EPI != EPI_NONE && live ? epi.bias[n] : 0.0f;
        float *yo = y + (int64_t)m * ldy + n;
        if constexpr (EPI == EPI_NONE) {
            if (live) *yo = acc;
        } else if constexpr (EPI == EPI_BIAS) {
            if (live) *yo = acc + bias;
        } else if constexpr (EPI == EPI_BIAS_GELU) {
            if (live) *yo = gelu_tanh(acc + bias);
        } else if constexpr (EPI == EPI_BIAS_RESID) {
            if (live) *yo = (acc + bias) + epi.resid[(int64_t)m * epi.ld_resid + n];
        } else if constexpr (EPI == EPI_GELU_Q81) {
            // columns past N quantize zeros: GELU(+0) = +0
            vr[m * 32 + c] = live ? gelu_tanh(acc + bias) : 0.0f;
        }
    }
    if constexpr (EPI == EPI_GELU_Q81) {
        static_assert(CW == 32, "one Q8_1 block of columns per workgroup");
        __syncthreads();
        // row m's block n0 / 32, as the MFMA forms' epilogue quantizes it
        if (tid < M) {
            const float *v = vr + tid * 32;
            float a = 0.0f;
            for (int k = 0; k < 32; ++k) a = fmaxf(a, fabsf(v[k]));
            const float d = a / 127.0f;
            const float inv = a != 0.0f ? 127.0f / a : 0.0f;
            int s = 0;
            uint32_t *qo = reinterpret_cast<uint32_t *>(epi.q_out8 + (int64_t)tid * epi.q_kpad + n0);
            for (int k = 0; k < 32; k += 4) {
                const int q0 = q8_round(v[k], inv), q1 = q8_round(v[k + 1], inv);
                const int q2 = q8_round(v[k + 2], inv), q3 = q8_round(v[k + 3], inv);
                qo[k / 4] = pack4_i8(q0, q1, q2, q3);
                s += q0 + q1 + q2 + q3;
            }
            epi.q_ds[(int64_t)tid * epi.q_ldds + n0 / QK] =
                (uint32_t)f32_to_f16_bits(d) | ((uint32_t)f32_to_f16_bits((float)s * d) << 16);
        }
    }
}

template <int CW, int EPI>
static hipError_t run_gemv(const WeightView &w, const int8_t *xq, const uint32_t *xds, int64_t ld_ds,
                           int64_t M, float *y, int64_t ldy, const EpiParams &epi, hipStream_t stream) {
    auto kern = k_gemv<CW, EPI>;
    static bool attr_set = false;  // idempotent; a racing second call repeats it harmlessly
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, GV_LDS_MAX);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const int64_t cols = EPI == EPI_GELU_Q81 ? epi.q_kpad : w.N;
    hipLaunchKernelGGL(kern, dim3((unsigned)((cols + CW - 1) / CW)), dim3(GV_NT),
                       (unsigned)gv_lds_bytes<CW>(M, w.K_pad), stream, xq, xds, ld_ds, w.qs, w.dT,
                       w.ldT, (int)w.K_pad, (int)M, (int)w.N, y, ldy, epi);
    return hipGetLastError();
}

// The GEMV form takes M <= 8 rows with a plain, bias, GELU, residual (not
// the position rows) or GELU -> Q8_1 epilogue and no K split, where its
// per-thread unrolls and LDS hold the sizes.
template <int CW>
static bool gv_fits(int64_t M, const WeightView &w) {
    const int64_t KB = w.K_pad / QK;
    return M <= GV_MAX_M && CW * KB <= GV_IT * GV_NT && M * KB <= GV_IT * GV_NT &&
           M * (w.K_pad / 16) <= GV_XIT * GV_NT && gv_lds_bytes<CW>(M, w.K_pad) <= GV_LDS_MAX;
}
static bool use_gemv(int64_t M, const WeightView &w, const EpiParams &epi) {
    switch (epi.kind) {
    case EPI_NONE: return epi.kb_split == 0 && gv_fits<8>(M, w);
    case EPI_BIAS:
    case EPI_BIAS_GELU: return gv_fits<8>(M, w);
    case EPI_BIAS_RESID: return epi.resid_rows == 0 && gv_fits<8>(M, w);
    case EPI_GELU_Q81: return gv_fits<32>(M, w);
    default: return false;
    }
}

template <int E>
static hipError_t run_gemv_epi(const WeightView &w, const int8_t *xq, const uint32_t *xds, int64_t ld_ds,
                               int64_t M, float *y, int64_t ldy, const EpiParams &epi, hipStream_t stream) {
    if constexpr (E == EPI_GELU_Q81)
        return run_gemv<32, E>(w, xq, xds, ld_ds, M, y, ldy, epi, stream);
    else if constexpr (E == EPI_NONE || E == EPI_BIAS || E == EPI_BIAS_GELU || E == EPI_BIAS_RESID)
        return run_gemv<8, E>(w, xq, xds, ld_ds, M, y, ldy, epi, stream);
    else
        return hipErrorInvalidValue;  // (use_gemv admits no other epilogue)
}

// Stage configurations: 4-block stages in a ring of 2.  Wide: 128 x 128
// tiles, two workgroups per CU, for GEMMs of enough tiles to fill the chip.
// Small: 64 x 128 tiles in the latency form, for GEMMs of fewer 128 x 128
// tiles than two per CU (M = 729: batch 1).  Each output's K order is the
// same in both, so the choice does not change a bit.  At M = 729 the small
// form takes out from 19.8 to 14.6 us and fc2 from 58.7 to 42.5 us; rings
// of 3 or 4 stages, 2-block stages and an imposed MFMA / VALU alternation
// measured slower.
#ifndef S2X_WIDE_TM
#define S2X_WIDE_TM 1
#endif
using Wide = gemm::Cfg<4, 2, 128, false, S2X_WIDE_TM>;
// The latency form's ring: four stages (three in flight) where its
// workgroups fit one per CU, three stages (two per CU) otherwise.  Where
// they fit one per CU, the plain / bias / residual epilogues (the out
// projection and fc2) run 8 waves of 32 x 32 outputs per 64 x 128 tile
// (Small4W): twice the waves, each with half the MFMA chain.  Where even
// those tiles number fewer than the CUs (out and fc2 at M = 729: 108 of
// them), 32 x 128 tiles of 4 such waves (Small4T) spread the rows over
// twice the workgroups: the same per-output K order, without splitting K.
using Small4 = gemm::Cfg<4, 4, 64, true>;
using Small4W = gemm::Cfg<4, 4, 64, true, 1, 1>;
using Small4T = gemm::Cfg<4, 4, 32, true, 1, 1>;
using Small3 = gemm::Cfg<4, 3, 64, true>;

template <int E>
static hipError_t run_small(const WeightView &w, const int8_t *xq, const uint32_t *xds, int64_t ld_ds,
                            int64_t M, float *y, int64_t ldy, const EpiParams &epi, hipStream_t stream);

static bool use_small(int64_t M, int64_t N) {
    return ((M + 127) / 128) * ((N + 127) / 128) < 2 * 256;
}
static bool small_ring4(int64_t M, int64_t N) { return ((M + 63) / 64) * ((N + 127) / 128) <= 256; }
static bool small_rows32(int64_t M, int64_t N) { return ((M + 63) / 64) * ((N + 127) / 128) < 256; }

hipError_t launch_gemm(const WeightView &w, const int8_t *xq, const uint32_t *xds, int64_t ld_ds,
                       int64_t M, float *y, int64_t ldy, const EpiParams &epi,
                       hipStream_t stream) {
    using C = Wide;
    if (M == 0 || w.N == 0) return hipSuccess;
    const int64_t KB = w.K_pad / QK;
    if (!w.qs || !w.dT || !xq || w.K_pad <= 0 || w.K_pad % QK || w.ldT < (w.N + 127) / 128 * 128 ||
        M > (1 << 30) || w.N > (1 << 30) || ((uintptr_t)xq & 15) || ((uintptr_t)w.qs & 15) ||
        ((uintptr_t)xds & 3) || (epi.kind != EPI_DUMP_I && (!xds || ld_ds < KB)) ||
        (int64_t)C::BM * KB * QK > 0x7fffffff || w.ldT * KB * 2 > 0x7fffffff ||
        C::BM * ld_ds * 4 > 0x7fffffff || C::BM * ldy * 4 > 0x7fffffff ||
        (epi.kb_split != 0 && (epi.kind != EPI_NONE || epi.kb_split < 0 || epi.y_split < M * ldy)))
        return hipErrorInvalidValue;
#define S2X_RUN(E)                                                                     \
    (use_gemv(M, w, epi) ? run_gemv_epi<E>(w, xq, xds, ld_ds, M, y, ldy, epi, stream)  \
     : !use_small(M, w.N) ? gemm::run<C, E>(w, xq, xds, ld_ds, M, y, ldy, epi, stream) \
                          : run_small<E>(w, xq, xds, ld_ds, M, y, ldy, epi, stream))
    switch (epi.kind) {
    case EPI_NONE: return S2X_RUN(EPI_NONE);
    case EPI_BIAS: return S2X_RUN(EPI_BIAS);
    case EPI_BIAS_GELU: return S2X_RUN(EPI_BIAS_GELU);
    case EPI_BIAS_RESID:
        if (!epi.resid || epi.ld_resid < w.N || epi.resid_rows < 0 ||
            (epi.resid_rows > 0 ? epi.resid_rows : C::BM) * epi.ld_resid * 4 > 0x7fffffff)
            return hipErrorInvalidValue;
        return S2X_RUN(EPI_BIAS_RESID);
    case EPI_DUMP_I:
        if (epi.dump_kb < 0 || epi.dump_kb >= KB) return hipErrorInvalidValue;
        return S2X_RUN(EPI_DUMP_I);
    case EPI_GELU_Q81:
        if (!epi.q_out8 || !epi.q_ds || !epi.bias || epi.q_kpad % QK || epi.q_kpad < w.N ||
            epi.q_kpad - w.N >= QK || epi.q_ldds < epi.q_kpad / QK ||
            ((uintptr_t)epi.q_out8 & 15) || ((uintptr_t)epi.q_ds & 3))
            return hipErrorInvalidValue;
        return S2X_RUN(EPI_GELU_Q81);
    case EPI_GELU_F16:
        if (!epi.h_out || !epi.bias || epi.h_kpad % QK || epi.h_kpad < w.N ||
            epi.h_kpad - w.N >= QK || epi.h_ld < epi.h_kpad)
            return hipErrorInvalidValue;
        return S2X_RUN(EPI_GELU_F16);
    case EPI_QKV:
        if (!epi.q || !epi.k || !epi.vt || !epi.rowmap || !epi.bias || epi.n_head <= 0 ||
            epi.d_head <= 0 || w.N != 3 * (int64_t)epi.n_head * epi.d_head || w.N >= (1 << 20))
            return hipErrorInvalidValue;
        return S2X_RUN(EPI_QKV);
    default: return hipErrorInvalidValue;
    }
#undef S2X_RUN
}

template <int E>
static hipError_t run_small(const WeightView &w, const int8_t *xq, const uint32_t *xds, int64_t ld_ds,
                            int64_t M, float *y, int64_t ldy, const EpiParams &epi, hipStream_t stream) {
    constexpr bool plain = E == EPI_NONE || E == EPI_BIAS || E == EPI_BIAS_GELU || E == EPI_BIAS_RESID ||
                           E == EPI_DUMP_I;
    if (!small_ring4(M, w.N)) return gemm::run<Small3, E>(w, xq, xds, ld_ds, M, y, ldy, epi, stream);
    if constexpr (plain) {
        if (small_rows32(M, w.N)) return gemm::run<Small4T, E>(w, xq, xds, ld_ds, M, y, ldy, epi, stream);
        return gemm::run<Small4W, E>(w, xq, xds, ld_ds, M, y, ldy, epi, stream);
    }
    return gemm::run<Small4, E>(w, xq, xds, ld_ds, M, y, ldy, epi, stream);
}

hipError_t launch_gemm_f16(const _Float16 *w16, int64_t K_pad, int64_t N, const _Float16 *x16,
                           int64_t M, float *y, int64_t ldy, const EpiParams &epi,
                           hipStream_t stream) {
    if (M == 0 || N == 0) return hipSuccess;
    if (!w16 || !x16 || !y || K_pad <= 0 || K_pad % QK || M > (1 << 30) || N > (1 << 30) ||
        ((uintptr_t)w16 & 15) || ((uintptr_t)x16 & 15) || (int64_t)gemm::CfgH::BM * K_pad * 2 > 0x7fffffff ||
        gemm::CfgH::BM * ldy * 4 > 0x7fffffff)
        return hipErrorInvalidValue;
    switch (epi.kind) {
    case EPI_NONE: return gemm::run_f16<EPI_NONE>(w16, K_pad, N, x16, M, y, ldy, epi, stream);
    case EPI_BIAS: return gemm::run_f16<EPI_BIAS>(w16, K_pad, N, x16, M, y, ldy, epi, stream);
    case EPI_BIAS_RESID:
        if (!epi.resid || epi.ld_resid < N || epi.resid_rows < 0 ||
            (epi.resid_rows > 0 ? epi.resid_rows : gemm::CfgH::BM) * epi.ld_resid * 4 > 0x7fffffff)
            return hipErrorInvalidValue;
        return gemm::run_f16<EPI_BIAS_RESID>(w16, K_pad, N, x16, M, y, ldy, epi, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace s2x
