// s2x_mmq16.hip -- Q8_0 (weights) x Q8_1 (activations) GEMM on gfx950 f16
// MFMA, bit-identical to the int8 formulation of s2x_mmq.hip:
//
//   Y[m, n] = sum_kb  fmaf(I_kb[m,n], dw[n,kb] * dx[m,kb], acc)   (kb in order)
//
// Why f16: with v_mfma_i32_32x32x32_i8 the per-block rescale costs three
// VALU instructions per output and block (convert, scale product, fma)
// against one 32-cycle MFMA per 1,024 outputs, i.e. 6x the VALU issue
// budget.  Here the quants are stored as f16 (exact integers, |q| <= 128):
//   * two v_mfma_f32_32x32x16_f16 give the block dot I as an exact f32
//     (products are integers < 2^14, partial sums integers < 2^20);
//   * the scale tile s[i][j] = dx[i] * dw[j] is one v_mfma_f32_32x32x8_f16
//     (two-register operands): A holds dx[row] and B holds dw[col] in k
//     slot 0, every other slot is zero, so each output is one exact
//     f16 x f16 product in f32.  The zero slots live in registers that are
//     cleared once; only the scale half-word is reloaded per block;
//   * the VALU does acc = fmaf(I, s, acc) -- the CPU's operation, one
//     instruction.
// Per 32x32 subtile and block: 3 MFMAs of 32 cycles each (96 cycles; the
// 32x32x8 form issues at the same rate as 32x32x16) against 16 VALU fmas
// (64 cycles): the matrix pipe bounds the kernel at 1/3 of the int8 peak.
//
// Tile: BM x 128 outputs per workgroup of BM/64 x 2 waves, each wave 64 x 64
// (2 x 2 subtiles).  One pipeline stage is one 32-value block of K: BM X rows
// and 128 W rows of 64 bytes plus their fp16 scales.  Stages are filled by
// LDS DMA (global_load_lds_dwordx4: each lane's 16 bytes land at the wave's
// LDS base + 16 * lane), so no staging registers; NS stages rotate, and the
// only waits are the wave's own DMA count (s_waitcnt vmcnt) and one barrier
// per block.  With PIPE the next stage's fragments are read from LDS into a
// second register set while the current one feeds the MFMAs.
//
// LDS layout of a stage's quant rows: 16-byte chunk c of row r is stored at
// chunk position c ^ ((r >> 2) & 3) of the row (64-byte rows): the MFMA
// operand reads (32 rows x one chunk per half-wave) then hit 16 distinct
// 16-byte bank groups per 16 lanes, which measured conflict-free on gfx950.
// The DMA side applies the same permutation on the global address each
// lane fetches.
//
// MFMA f16 32x32x16 layout: lane l supplies row (l & 31) of A and column
// (l & 31) of B, k-slots 8*(l >> 5) .. +7; result register r of lane l holds
// row 8*(r/4) + 4*(l/32) + (r%4), column (l & 31).
#include "s2x_device.h"
#include "s2x_kernels.h"

#include <type_traits>

namespace s2x {
namespace mmq16 {

constexpr int GM = 8;         // tile-row group of the tile order
constexpr int BUF_DW3 = 0x00020000;  // buffer resource word 3: raw 32-bit dwords

template <int BM_, int NS_, bool PIPE_, int TM_ = 2, bool SKEW_ = true, bool I8_ = false,
          int TN_ = 2, int KS_ = 1>
struct Cfg {
    static constexpr int BM = BM_, NS = NS_, TM = TM_;  // TM: 32-row subtiles per wave
    static constexpr int KS = KS_;  // K blocks per stage (one barrier per stage)
    static constexpr int TN = TN_;                      // TN: 32-column subtiles per wave
    static constexpr int BN = 2 * 32 * TN;              // two waves along N
    static constexpr bool I8 = I8_;      // int8 quants, v_mfma_i32_32x32x32_i8 block dots
    static constexpr int ROWB = QK * (I8 ? 1 : 2);  // bytes of one block of one row
    static constexpr int CH = ROWB / 16;            // 16-byte chunks per row and block
    // Chunk permutation of tile row r (only r's low 5 bits matter).  A
    // fragment read has each lane take one 16-byte chunk of its own row;
    // the permutation spreads the chunks of rows r, r + 4, r + 8, r + 12
    // over distinct LDS banks.
    static __device__ __forceinline__ int swz(int r) {
        return CH == 2 ? ((r >> 2) ^ (r >> 3)) & 1 : (r >> 2) & (CH - 1);
    }
    static constexpr bool PIPE = PIPE_;  // next block's fragments read during this block's MFMAs
    static constexpr bool SKEW = SKEW_;  // a subtile's fmas issued after the next one's MFMAs
    static constexpr int WGM = BM / (32 * TM);          // waves along M (2 along N)
    static constexpr int NWAVE = WGM * 2;
    static constexpr int NT = NWAVE * WAVE;
    // quant DMA instructions per thread and stage: the stage's X chunks
    // then its W chunks, NT per instruction (each wave's 64 are all X or all W)
    static constexpr int QI = (BM + BN) * CH / NT;
    static constexpr int X_BYTES = BM * ROWB;
    static constexpr int DX_OFF = X_BYTES + BN * ROWB;  // BM fp16 X scales
    static constexpr int DW_OFF = DX_OFF + BM * 2;      // BN fp16 W scales
    static constexpr int Z_OFF = DW_OFF + BN * 2;       // 16 zero bytes
    static constexpr int STAGE = Z_OFF + 16;
    // the stage ring, or the epilogues' 32 x 144-byte scratch rows per wave
    static constexpr int LDS =
        NS * KS * STAGE > NWAVE * 32 * 144 ? NS * KS * STAGE : NWAVE * 32 * 144;
    static_assert(BM % (32 * TM) == 0 && (TM == 1 || TM == 2) && (TN == 1 || TN == 2) && QI >= 1 &&
                      (BM + BN) * CH == QI * NT && (BM * CH) % WAVE == 0 && BM / 8 <= WAVE &&
                      BN / 8 <= WAVE && (!I8 || TM == 1),
                  "config");
    static_assert(NS >= 2 && NS <= (PIPE ? 4 : 8) && KS >= 1 && (KS == 1 || !PIPE) &&
                      (NS - 2) * KS <= 6,
                  "wait table / unroll");
};

typedef __attribute__((address_space(3))) void lds_void;

template <int TM, int TN, bool I8>
struct FragTM {
    // quant operands: f16 [subtile][k half] (two 32x32x16 MFMAs per block)
    // or int8 [subtile] (one 32x32x32 MFMA per block)
    std::conditional_t<I8, v4i, v8h> a[TM][I8 ? 1 : 2], b[TN][I8 ? 1 : 2];
    // scale-tile operands (32x32x8 f16 MFMA, k slots 0..3 on lanes 0..31):
    // dword 0 holds the fp16 bits of the row / column scale (0 on lanes
    // 32..63), dword 1 stays zero for the whole loop, so only dword 0 is
    // reloaded per block
    v2i sx[TM], sw[TN];
    __device__ void zero_scales() {
        for (int a = 0; a < TM; ++a) sx[a] = v2i{0, 0};
        for (int b = 0; b < TN; ++b) sw[b] = v2i{0, 0};
    }
};

// 16 bytes per lane from buffer r at voffset + soffset into LDS at
// lds_wave_base + 16 * lane; reads past the buffer's size return zeros.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                      uint8_t *lds_wave_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds_wave_base, 16, voff, soff, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// This wave's LDS reads done, then the workgroup barrier (no vmcnt wait:
// later stages' DMA stays in flight).
__device__ __forceinline__ void block_sync_lds() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Wait until a stage has landed, given `after` later stages already issued
// and L DMA instructions per stage from this wave.
template <int L>
__device__ __forceinline__ void wait_after(int after) {
    switch (after) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<L>(); break;
    case 2: wait_vm<2 * L>(); break;
    case 3: wait_vm<3 * L>(); break;
    case 4: wait_vm<4 * L>(); break;
    case 5: wait_vm<5 * L>(); break;
    default: wait_vm<6 * L>(); break;
    }
}

// f(integral_constant<int, J>) for J = J0 .. J1 - 1, in order
template <int J0, int J1, class F>
__device__ __forceinline__ void unroll_const(F &&f) {
    if constexpr (J0 < J1) {
        f(std::integral_constant<int, J0>{});
        unroll_const<J0 + 1, J1>(f);
    }
}

// a / b for 0 <= a < 2^20 and b >= 1, exact: the float estimate a * (1/b)
// is within a/b * 2^-23 <= 1/8 of a/b, so one correction either way suffices
__device__ __forceinline__ int small_div(int a, int b, float inv_b) {
    int q = (int)((float)a * inv_b);
    const int r = a - q * b;
    q += (r >= b) - (r < 0);
    return q;
}

// Waves 0 and 1 also fetch the X and the W scales.
template <class C>
__device__ __forceinline__ void wait_stage(bool scale_wave, int after) {
    if (scale_wave)
        wait_after<C::QI + 1>(after);
    else
        wait_after<C::QI>(after);
}

template <class C, int EPI>
__global__ __launch_bounds__(C::NT) __attribute__((amdgpu_waves_per_eu(C::TM == 1 ? 4 : 2))) void k_mmq16(
    const uint8_t *__restrict__ xq, const uint16_t *__restrict__ xdT, int64_t ld_dx,
    const uint8_t *__restrict__ wq, const uint16_t *__restrict__ wdT, int64_t ld_dw, int M,
    int N, int KB, float *__restrict__ y, int64_t ldy, EpiParams epi) {
    constexpr int BM = C::BM, BN = C::BN, NS = C::NS, NT = C::NT, TM = C::TM, TN = C::TN;
    constexpr int ROWB = C::ROWB, CH = C::CH;
    using Frag = FragTM<TM, TN, C::I8>;
    extern __shared__ __align__(16) uint8_t lds[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar registers
    const int wm = wave >> 1, wn = wave & 1;
    const int m_tiles = (M + BM - 1) / BM, n_tiles = (N + BN - 1) / BN;
    int tmi, tni;
    tile_coords<GM>(blockIdx.x, gridDim.x, m_tiles, n_tiles, tmi, tni);
    const int m0 = tmi * BM, n0 = tni * BN;
    const int64_t K_pad = (int64_t)KB * QK;
    const int64_t row_bytes = K_pad * (C::I8 ? 1 : 2);

    // Buffers over this tile's rows: rows past M / N read as zeros (their
    // outputs are never stored).  Position p (16-byte unit) of a stage's X
    // (then W) rows holds chunk (p % CH) ^ C::swz(row) of row
    // p / CH.
    const auto clip = [](int64_t bytes) { return (int)min(bytes, (int64_t)0x7fffffff); };
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(xq + (int64_t)m0 * row_bytes), (short)0, clip((int64_t)(M - m0) * row_bytes), BUF_DW3);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(wq + (int64_t)n0 * row_bytes), (short)0, clip((int64_t)(N - n0) * row_bytes), BUF_DW3);
    uint32_t qv[C::QI];
#pragma unroll
    for (int i = 0; i < C::QI; ++i) {
        const int p = i * NT + tid;
        const int pr = p < BM * CH ? p : p - BM * CH;  // position within X or W
        const int row = pr / CH, chunk = (pr % CH) ^ C::swz(row);
        qv[i] = (uint32_t)(row * row_bytes) + (uint32_t)chunk * 16;
    }
    // wave 0: X scales (BM/8 lanes x 8), wave 1: W scales (BN/8 lanes x 8)
    const bool scale_wave = wave < 2;
    const bool s_lane = lane < (wave == 0 ? BM / 8 : BN / 8);
    const __amdgpu_buffer_rsrc_t sr =
        wave == 0 ? __builtin_amdgcn_make_buffer_rsrc((void *)(xdT + m0), (short)0,
                                                      clip((KB * ld_dx - m0) * 2), BUF_DW3)
                  : __builtin_amdgcn_make_buffer_rsrc((void *)(wdT + n0), (short)0,
                                                      clip((KB * ld_dw - n0) * 2), BUF_DW3);
    const uint32_t s_stride = (uint32_t)((wave == 0 ? ld_dx : ld_dw) * 2);
    const int s_dst = wave == 0 ? C::DX_OFF : C::DW_OFF;

    // Fill stage buffer `buf` with block kb.  buf is free: every wave has
    // finished reading it before the last barrier.
    auto issue = [&](int kb, int buf) {
        uint8_t *sb = lds + buf * C::STAGE;
        const uint32_t koff = (uint32_t)kb * ROWB;
#pragma unroll
        for (int i = 0; i < C::QI; ++i) {
            const int p0 = i * NT + wave * 64;  // wave-uniform: the 64 chunks are X or W
            dma16(p0 < BM * CH ? xr : wr, qv[i], koff, sb + p0 * 16);
        }
        if (scale_wave && s_lane) dma16(sr, (uint32_t)lane * 16, (uint32_t)kb * s_stride, sb + s_dst);
    };

    // the zero words read by lanes 32..63 for the scale operands
    if (tid < NS * C::KS) *reinterpret_cast<v4i *>(lds + tid * C::STAGE + C::Z_OFF) = v4i{0, 0, 0, 0};

    float acc[TM][TN][16];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

    const int lr = lane & 31, lh = lane >> 5;
    const int xrow0 = wm * 32 * TM + lr, wcol0 = wn * 32 * TN + lr;
    // the epilogue's bias of this lane's columns, fetched before the main
    // loop so that its latency is hidden (0 past N)
    float bias_v[TN];
#pragma unroll
    for (int b = 0; b < TN; ++b) {
        const int n = n0 + wcol0 + b * 32;
        bias_v[b] = EPI != EPI_NONE && EPI != EPI_DUMP_I && n < N ? epi.bias[n] : 0.0f;
    }
    const int sw = C::swz(lr);  // chunk permutation of the rows this lane reads
    // k slots 8 lh .. 8 lh + 7 (f16: of each 16-value half) / 16 lh .. +15 (int8)
    const int c0 = (lh ^ sw) * 16, c1 = ((2 + lh) ^ sw) * 16;
    const int xo = xrow0 * ROWB, wo = C::X_BYTES + wcol0 * ROWB;
    // scale operands: k slot 0 (lanes 0..31) holds the scale, the rest zeros
    const int dxo0 = lh ? C::Z_OFF : C::DX_OFF + xrow0 * 2;
    const int dxo1 = lh ? C::Z_OFF : C::DX_OFF + (xrow0 + 32 * (TM - 1)) * 2;
    const int dwo0 = lh ? C::Z_OFF : C::DW_OFF + wcol0 * 2;
    const int dwo1 = lh ? C::Z_OFF : C::DW_OFF + (wcol0 + 32 * (TN - 1)) * 2;

    auto load_frag = [&](const uint8_t *sb, Frag &f) {
#pragma unroll
        for (int a = 0; a < TM; ++a) {
            if constexpr (C::I8) {
                f.a[a][0] = *reinterpret_cast<const v4i *>(sb + xo + a * 32 * ROWB + c0);
            } else {
                f.a[a][0] = *reinterpret_cast<const v8h *>(sb + xo + a * 32 * ROWB + c0);
                f.a[a][1] = *reinterpret_cast<const v8h *>(sb + xo + a * 32 * ROWB + c1);
            }
        }
        f.sx[0][0] = *reinterpret_cast<const uint16_t *>(sb + dxo0);
        if constexpr (TM == 2) f.sx[1][0] = *reinterpret_cast<const uint16_t *>(sb + dxo1);
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            if constexpr (C::I8) {
                f.b[b][0] = *reinterpret_cast<const v4i *>(sb + wo + b * 32 * ROWB + c0);
            } else {
                f.b[b][0] = *reinterpret_cast<const v8h *>(sb + wo + b * 32 * ROWB + c0);
                f.b[b][1] = *reinterpret_cast<const v8h *>(sb + wo + b * 32 * ROWB + c1);
            }
        }
        f.sw[0][0] = *reinterpret_cast<const uint16_t *>(sb + dwo0);
        if constexpr (TN == 2) f.sw[1][0] = *reinterpret_cast<const uint16_t *>(sb + dwo1);
    };

    // One block of K.  Subtile k = 2a + b gets I (f16: two MFMAs, exact f32;
    // int8: one MFMA, exact int32) and the scale tile (one MFMA);
    // acc = fmaf(I, s, acc) for subtile k runs after subtile k+1's MFMAs are
    // issued, and subtile 3's in the next block, so the VALU work overlaps
    // the matrix pipe.  Each acc element still receives its fmas in block
    // order.
    using IT = std::conditional_t<C::I8, v16i, v16f>;
    IT Ip;
    v16f Sp;
    bool pending = false;
    auto mma = [&](const Frag &f) {
        const v16f zero = {};
        const v16i zero_i = {};
#pragma unroll
        for (int k = 0; k < TM * TN; ++k) {
            const int a = k / TN, b = k % TN;
            IT I;
            v16f S;
            if constexpr (C::I8) {
                I = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[a][0], f.b[b][0], zero_i, 0, 0, 0);
                S = __builtin_amdgcn_mfma_f32_32x32x8f16(
                    __builtin_bit_cast(v4h, f.sx[a]), __builtin_bit_cast(v4h, f.sw[b]), zero, 0, 0, 0);
            } else {
                I = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[a][0], f.b[b][0], zero, 0, 0, 0);
                S = __builtin_amdgcn_mfma_f32_32x32x8f16(
                    __builtin_bit_cast(v4h, f.sx[a]), __builtin_bit_cast(v4h, f.sw[b]), zero, 0, 0, 0);
                I = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[a][1], f.b[b][1], I, 0, 0, 0);
            }
            if constexpr (!C::SKEW) {
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[a][b][r] = fmaf((float)I[r], S[r], acc[a][b][r]);
                continue;
            }
            const int pk = (k + TM * TN - 1) % (TM * TN), pa = pk / TN, pb = pk % TN;
            if (k > 0 || pending) {
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[pa][pb][r] = fmaf((float)Ip[r], Sp[r], acc[pa][pb][r]);
            }
            Ip = I;
            Sp = S;
            // issue order: each MFMA followed by its share of the previous
            // subtile's VALU work, so a wave alone keeps the matrix pipe fed
            if (k > 0 || pending) {
                if constexpr (C::I8) {  // 2 MFMAs, 16 converts + 16 fmas
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
                } else {  // 3 MFMAs, 16 fmas
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
                }
            }
        }
        pending = true;
    };

    if constexpr (C::KS > 1) {
        // Stages of KS blocks (KS sub-buffers each), NS-1 stages in flight,
        // one wait + barrier per stage; the blocks of a stage are separated
        // by scheduling barriers so that only one block's fragments are live.
        constexpr int KS = C::KS;
        const int n_stages = (KB + KS - 1) / KS;
        auto issue_stage = [&](int st, int sbuf) {
#pragma unroll
            for (int j = 0; j < KS; ++j)
                if (st * KS + j < KB) issue(st * KS + j, sbuf * KS + j);
        };
        const int npro = min(NS - 1, n_stages);
        for (int st = 0; st < npro; ++st) issue_stage(st, st);
        Frag F;
        F.zero_scales();
        auto stage = [&](int st, auto bufc) {
            constexpr int sbuf = decltype(bufc)::value;
            // blocks issued after this stage's: those of the next
            // min(NS - 2, n_stages - 1 - st) stages (the last one may be short)
            const int later = min(st + NS - 1, n_stages) - (st + 1);
            const int later_blocks = later <= 0 ? 0 : min(later * KS, KB - (st + 1) * KS);
            wait_stage<C>(scale_wave, later_blocks);
            block_sync_lds();
            if (st + NS - 1 < n_stages) issue_stage(st + NS - 1, (sbuf + NS - 1) % NS);
            unroll_const<0, KS>([&](auto jc) {
                constexpr int j = decltype(jc)::value;
                if (st * KS + j < KB) {
                    load_frag(lds + (sbuf * KS + j) * C::STAGE, F);
                    mma(F);
                }
                __builtin_amdgcn_sched_barrier(0);
            });
        };
        for (int st = 0; st < n_stages; st += NS) {
            unroll_const<0, NS>([&](auto jc) {
                constexpr int j = decltype(jc)::value;
                if (st + j < n_stages) stage(st + j, jc);
            });
        }
    } else if constexpr (!C::PIPE) {
        // NS-1 blocks in flight; stage s+NS-1 refills the buffer of stage
        // s-1.  The stage loop is unrolled NS times so each LDS read's stage
        // offset is an instruction immediate.
        const int npro = min(NS - 1, KB);
        for (int s = 0; s < npro; ++s) issue(s, s);
        Frag F;
        F.zero_scales();
        auto step = [&](int s, auto bufc) {
            constexpr int buf = decltype(bufc)::value;
            wait_stage<C>(scale_wave, min(NS - 2, KB - 1 - s));
            block_sync_lds();
            if (s + NS - 1 < KB) issue(s + NS - 1, (buf + NS - 1) % NS);
            load_frag(lds + buf * C::STAGE, F);
            mma(F);
        };
        for (int s = 0; s < KB; s += NS) {
            unroll_const<0, NS>([&](auto jc) {
                constexpr int j = decltype(jc)::value;
                if (s + j < KB) step(s + j, jc);
            });
        }
    } else {
        // NS blocks in flight; block s+1's fragments are read from LDS while
        // block s's are in the MFMAs, and block s+NS refills the buffer of s
        // (read into registers during the previous step).  Unrolled 2*NS
        // times: stage offsets are immediates and the fragment sets alternate.
        const int npro = min(NS, KB);
        for (int s = 0; s < npro; ++s) issue(s, s);
        wait_stage<C>(scale_wave, npro - 1);
        block_sync_lds();
        Frag F0, F1;
        F0.zero_scales();
        F1.zero_scales();
        load_frag(lds, F0);
        auto step = [&](int s, auto bufc, Frag &cur, Frag &nxt) {
            constexpr int buf = decltype(bufc)::value;  // buffer of block s
            if (s + 1 < KB) {
                wait_stage<C>(scale_wave, min(NS - 2, KB - 2 - s));
                block_sync_lds();
                load_frag(lds + ((buf + 1) % NS) * C::STAGE, nxt);
                if (s + NS < KB) issue(s + NS, buf);
            }
            mma(cur);
        };
        static_assert(NS == 2 || NS == 3 || NS == 4, "unroll");
        for (int s = 0; s < KB; s += 2 * NS) {
            step(s, std::integral_constant<int, 0>{}, F0, F1);
            if (s + 1 < KB) step(s + 1, std::integral_constant<int, 1 % NS>{}, F1, F0);
            if (s + 2 < KB) step(s + 2, std::integral_constant<int, 2 % NS>{}, F0, F1);
            if (s + 3 < KB) step(s + 3, std::integral_constant<int, 3 % NS>{}, F1, F0);
            if constexpr (NS > 2) {
                if (s + 4 < KB) step(s + 4, std::integral_constant<int, 4 % NS>{}, F0, F1);
                if (s + 5 < KB) step(s + 5, std::integral_constant<int, 5 % NS>{}, F1, F0);
            }
            if constexpr (NS > 3) {
                if (s + 6 < KB) step(s + 6, std::integral_constant<int, 6 % NS>{}, F0, F1);
                if (s + 7 < KB) step(s + 7, std::integral_constant<int, 7 % NS>{}, F1, F0);
            }
        }
    }
    if constexpr (C::SKEW) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[TM - 1][TN - 1][r] = fmaf((float)Ip[r], Sp[r], acc[TM - 1][TN - 1][r]);
    }
    // The stage loop's waits are inline asm, which the compiler's wait
    // placement cannot see: this vmcnt(0) (expcnt / lgkmcnt left alone) --
    // free here, nothing is in flight -- tells it that bias_v has arrived,
    // so the epilogue's stores are not each preceded by a vmcnt(0).
    __builtin_amdgcn_s_waitcnt(0x0F70);

    if constexpr (EPI == EPI_GELU_Q81) {
        // GELU(mm + bias), then Q8_1 exactly as k_quantize_q8_1 over rows of
        // q_kpad values (columns >= N are zeros).  A wave's 32 x 32 subtile is
        // one quant block per row: it goes through LDS so that lane pairs own
        // a row (16 values each); the stage buffers are free after a barrier.
        constexpr int P = 36;  // floats per scratch row (16-byte aligned rows)
        static_assert(C::NWAVE * 32 * P * 4 <= C::LDS, "epilogue scratch fits the stages");
        __syncthreads();
        float *scr = reinterpret_cast<float *>(lds) + wave * 32 * P;
        const int row = lane >> 1, half = lane & 1;
        const int m = m0 + wm * 32 + row;
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int nb = n0 + wn * 32 * TN + b * 32;  // first column of this quant block
            if (nb >= epi.q_kpad) continue;        // wave-uniform
            const int n = nb + lr;
#pragma unroll
            for (int r = 0; r < 16; ++r)
                scr[(8 * (r >> 2) + 4 * lh + (r & 3)) * P + lr] =
                    n < N ? gelu_tanh(acc[0][b][r] + bias_v[b]) : 0.0f;
            float v[16];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const v4f t = *reinterpret_cast<const v4f *>(scr + row * P + half * 16 + 4 * j);
                v[4 * j] = t[0]; v[4 * j + 1] = t[1]; v[4 * j + 2] = t[2]; v[4 * j + 3] = t[3];
            }
            float a = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) a = fmaxf(a, fabsf(v[j]));
            a = fmaxf(a, dpp_f<0xb1>(a));  // partner lane (xor 1)
            const float d = a / 127.0f;
            const float inv = a != 0.0f ? 127.0f / a : 0.0f;
            int qi[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) qi[j] = q8_round(v[j], inv);
            if (m < M) {
                const int64_t off = (int64_t)m * epi.q_kpad + nb + half * 16;
                if constexpr (C::I8) {
                    *reinterpret_cast<uint4 *>(epi.q_out8 + off) =
                        make_uint4(pack4_i8(qi[0], qi[1], qi[2], qi[3]), pack4_i8(qi[4], qi[5], qi[6], qi[7]),
                                   pack4_i8(qi[8], qi[9], qi[10], qi[11]),
                                   pack4_i8(qi[12], qi[13], qi[14], qi[15]));
                } else {
                    v8h q0, q1;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        q0[j] = (_Float16)qi[j];
                        q1[j] = (_Float16)qi[8 + j];
                    }
                    v8h *dst = reinterpret_cast<v8h *>(epi.q_out + off);
                    dst[0] = q0;
                    dst[1] = q1;
                }
                if (half == 0) epi.q_dT[(int64_t)(nb / QK) * epi.q_ld + m] = f32_to_f16_bits(d);
            }
        }
        return;
    }

    if constexpr (EPI == EPI_QKV) {
        // (mm + bias) in f32, then f16, into Q / K [seg][head][pos][d_pad] or
        // V^T [seg][head][dv_pad][pos]; padding slots are not written
        const int H = epi.n_head * epi.d_head;
        const float inv_dh = 1.0f / (float)epi.d_head;
        if constexpr (TM == 1 && TN == 2) {
        if (n0 + BN <= 2 * H && H % BN == 0 && epi.d_head % 8 == 0 && epi.d_pad % 8 == 0) {
            // a Q or K tile (the q|k|v boundaries fall on tile edges): the
            // wave's 32 x 64 f16 tile goes through LDS so that each 8-column
            // chunk of a row -- 8 consecutive d of one head -- leaves as one
            // 16-byte store
            constexpr int P = 72;  // halves per scratch row (16-byte aligned)
            static_assert(C::NWAVE * 32 * P * 2 <= C::LDS, "epilogue scratch fits the stages");
            __syncthreads();
            _Float16 *scr = reinterpret_cast<_Float16 *>(lds) + wave * 32 * P;
#pragma unroll
            for (int b = 0; b < 2; ++b) {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    scr[(8 * (r >> 2) + 4 * lh + (r & 3)) * P + b * 32 + lr] =
                        f32_to_f16(acc[0][b][r] + bias_v[b]);
            }
            _Float16 *dst0 = n0 < H ? epi.q : epi.k;
            int rmv[4];  // row map entries, all loaded before the first store
#pragma unroll
            for (int i = 0; i < 4; ++i)
                rmv[i] = epi.rowmap[min(m0 + wm * 32 + ((lane + 64 * i) >> 3), M - 1)];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int id = lane + 64 * i, row = id >> 3, c = (id & 7) * 8;
                const int m = m0 + wm * 32 + row, n = n0 + wn * 64 + c;
                if (m >= M || n >= N) continue;
                const int hd = n0 < H ? n : n - H;  // the tile is all Q or all K
                const int h = small_div(hd, epi.d_head, inv_dh), d = hd - h * epi.d_head;
                const int rm = rmv[i];
                const int64_t sh = (int64_t)(rm >> 16) * epi.n_head + h;
                const v8h v = *reinterpret_cast<const v8h *>(scr + row * P + c);
                *reinterpret_cast<v8h *>(dst0 + (sh * epi.len_pad + (rm & 0xffff)) * epi.d_pad + d) = v;
            }
            return;
        }
        constexpr int VT_PT = 40;  // halves per V^T scratch column (below)
        constexpr bool VT_FITS = C::NWAVE * 64 * VT_PT * 2 <= C::LDS;
        if (VT_FITS && n0 >= 2 * H && H % BN == 0) {
            // a V tile: V^T rows are positions, so the wave's 32 x 64 tile
            // goes through LDS transposed (column-major, rows shifted by the
            // first position's offset within its 8-position chunk) and each
            // lane writes one column -- one d of one head: up to 32
            // consecutive positions -- as 16-byte stores where the
            // destination is 16-byte aligned, 2-byte stores at the ends
            // halves per scratch column: shift <= 7 + 32 rows; 80-byte columns
            // keep 16-byte alignment and put lanes 0..31 on 16 bank groups
            // (configurations whose LDS is smaller take the generic path)
            constexpr int PT = VT_PT;
            const int mw = m0 + wm * 32;
            const int rows = min(32, M - mw);  // wave-uniform, may be <= 0
            int rm_first = 0, rm_last = 0;
            if (rows > 0) {
                rm_first = epi.rowmap[mw];
                rm_last = epi.rowmap[mw + rows - 1];
            }
            // one segment, consecutive positions: the common case
            const bool run = rows > 0 && (rm_last >> 16) == (rm_first >> 16) &&
                             (rm_last & 0xffff) - (rm_first & 0xffff) == rows - 1;
            const int shift = run ? (rm_first & 0xffff) & 7 : 0;
            __syncthreads();
            _Float16 *scr = reinterpret_cast<_Float16 *>(lds) + wave * 64 * PT;
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        scr[(b * 32 + lr) * PT + shift + 8 * q + 4 * lh + j] =
                            f32_to_f16(acc[0][b][4 * q + j] + bias_v[b]);
            __syncthreads();
            const int n = n0 + wn * 64 + lane;
            if (rows <= 0 || n >= N) return;
            const int hd = n - 2 * H, h = small_div(hd, epi.d_head, inv_dh);
            const int d = hd - h * epi.d_head;
            const _Float16 *col = scr + lane * PT;
            if (run) {
                const int64_t sh = (int64_t)(rm_first >> 16) * epi.n_head + h;
                _Float16 *dst = epi.vt + (sh * epi.dv_pad + d) * epi.len_pad + (rm_first & 0xffff) - shift;
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
                    const int rm = epi.rowmap[mw + i];
                    const int64_t sh = (int64_t)(rm >> 16) * epi.n_head + h;
                    epi.vt[(sh * epi.dv_pad + d) * epi.len_pad + (rm & 0xffff)] = col[i];
                }
            }
            return;
        }
        }
        // the row map of this lane's rows, all loaded before the first store
        int rmv[TM][16];
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 32 * TM + a * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                rmv[a][r] = epi.rowmap[min(m, M - 1)];
            }
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int n = n0 + wcol0 + b * 32;
            if (n >= N) continue;
            const int part = small_div(n, H, 1.0f / (float)H), hd = n - part * H;
            const int h = small_div(hd, epi.d_head, inv_dh), d = hd - h * epi.d_head;
            _Float16 *dst = part == 0 ? epi.q : part == 1 ? epi.k : epi.vt;
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm * 32 * TM + a * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                    if (m >= M) continue;
                    const int rm = rmv[a][r];
                    const int64_t sh = (int64_t)(rm >> 16) * epi.n_head + h;
                    const int pos = rm & 0xffff;
                    const int64_t off = part < 2 ? (sh * epi.len_pad + pos) * epi.d_pad + d
                                                 : (sh * epi.dv_pad + d) * epi.len_pad + pos;
                    dst[off] = f32_to_f16(acc[a][b][r] + bias_v[b]);
                }
        }
        return;
    }

    // (mm + bias) [GELU | + residual] in acc, every residual load issued
    // before the first store (y may be the residual itself: each element is
    // read before it is written, and by the lane that writes it)
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int n = n0 + wcol0 + b * 32;
            const int nc = min(n, N - 1);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float v = acc[a][b][r];
                if (EPI == EPI_BIAS) {
                    v = v + bias_v[b];
                } else if (EPI == EPI_BIAS_GELU) {
                    v = gelu_tanh(v + bias_v[b]);
                } else if (EPI == EPI_BIAS_RESID) {
                    const int m = m0 + wm * 32 * TM + a * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                    const int mc = min(m, M - 1);
                    const int rm = epi.resid_rows > 0 && epi.resid_rows < M ? mc % (int)epi.resid_rows : mc;
                    v = (v + bias_v[b]) + epi.resid[(int64_t)rm * epi.ld_resid + nc];
                }
                acc[a][b][r] = v;
            }
        }
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int n = n0 + wcol0 + b * 32;
            if (n >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 32 * TM + a * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (m < M) y[(int64_t)m * ldy + n] = acc[a][b][r];
            }
        }
}

template <class C, int EPI>
hipError_t run(const WeightView &w, const void *xq, const uint16_t *xdT, int64_t ld_dx,
               int64_t M, float *y, int64_t ldy, const EpiParams &epi, hipStream_t stream) {
    const int m_tiles = (int)((M + C::BM - 1) / C::BM), n_tiles = (int)((w.N + C::BN - 1) / C::BN);
    auto kern = k_mmq16<C, EPI>;
    static bool attr_set = false;  // idempotent; a racing second call repeats it harmlessly
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 C::LDS);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const void *wq = C::I8 ? (const void *)w.qs : (const void *)w.qh;
    hipLaunchKernelGGL(kern, dim3(m_tiles * n_tiles), dim3(C::NT), C::LDS, stream,
                       reinterpret_cast<const uint8_t *>(xq), xdT, ld_dx,
                       reinterpret_cast<const uint8_t *>(wq), w.dT, w.ldT, (int)M, (int)w.N,
                       (int)(w.K_pad / QK), y, ldy, epi);
    return hipGetLastError();
}

template <class C>
hipError_t dispatch(const WeightView &w, const void *xh, const uint16_t *xdT, int64_t ld_dx,
                    int64_t M, float *y, int64_t ldy, const EpiParams &epi, hipStream_t stream) {
    switch (epi.kind) {
    case EPI_NONE: return run<C, EPI_NONE>(w, xh, xdT, ld_dx, M, y, ldy, epi, stream);
    case EPI_BIAS: return run<C, EPI_BIAS>(w, xh, xdT, ld_dx, M, y, ldy, epi, stream);
    case EPI_BIAS_GELU: return run<C, EPI_BIAS_GELU>(w, xh, xdT, ld_dx, M, y, ldy, epi, stream);
    case EPI_BIAS_RESID: return run<C, EPI_BIAS_RESID>(w, xh, xdT, ld_dx, M, y, ldy, epi, stream);
    case EPI_GELU_Q81:
        if (C::TM != 1 || !(C::I8 ? (void *)epi.q_out8 : (void *)epi.q_out) || !epi.q_dT || !epi.bias || epi.q_kpad % QK ||
            epi.q_kpad < w.N || epi.q_kpad - w.N >= QK || epi.q_ld < mmq16_ld_dx(M) ||
            (reinterpret_cast<uintptr_t>(C::I8 ? (void *)epi.q_out8 : (void *)epi.q_out) & 15))
            return hipErrorInvalidValue;
        return run<C, EPI_GELU_Q81>(w, xh, xdT, ld_dx, M, y, ldy, epi, stream);
    case EPI_QKV:
        if (!epi.q || !epi.k || !epi.vt || !epi.rowmap || !epi.bias || epi.n_head <= 0 ||
            epi.d_head <= 0 || w.N != 3 * (int64_t)epi.n_head * epi.d_head || w.N >= (1 << 20))
            return hipErrorInvalidValue;
        return run<C, EPI_QKV>(w, xh, xdT, ld_dx, M, y, ldy, epi, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace mmq16

static bool mmq_args_ok(const WeightView &w, const void *xq, const uint16_t *xdT, int64_t ld_dx,
                        int64_t M) {
    return w.dT && xq && xdT && ld_dx >= mmq16_ld_dx(M) && !(ld_dx & 7) &&
           w.ldT >= mmq16_ld_dw(w.N) && !(w.ldT & 7) && !(w.K_pad % QK) && w.K_pad != 0 &&
           !(reinterpret_cast<uintptr_t>(xq) & 15) && !(reinterpret_cast<uintptr_t>(xdT) & 15);
}

namespace mmq16 {

// Workgroups of config C resident at once on the current device.
template <class C>
int64_t resident_tiles() {
    static int cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (!cached[dev]) {
        int cus = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &per_cu, reinterpret_cast<const void *>(k_mmq16<C, EPI_NONE>), C::NT, C::LDS) !=
                hipSuccess)
            return 0;
        cached[dev] = cus * per_cu;
    }
    return cached[dev];
}

// The epilogue of rows [r, ...) of a GEMM as a GEMM of its own; false when
// the row shift cannot be expressed (a residual read modulo resid_rows).
inline bool shift_rows(const EpiParams &e, int64_t r, float *&y, int64_t ldy, EpiParams &out) {
    out = e;
    if (y) y += r * ldy;
    switch (e.kind) {
    case EPI_BIAS_RESID:
        if (e.resid_rows > 0) return r % e.resid_rows == 0;
        out.resid = e.resid + r * e.ld_resid;
        return true;
    case EPI_QKV: out.rowmap = e.rowmap + r; return true;
    case EPI_GELU_Q81:
        if (e.q_out) out.q_out = e.q_out + r * e.q_kpad;
        if (e.q_out8) out.q_out8 = e.q_out8 + r * e.q_kpad;
        out.q_dT = e.q_dT + r;
        return true;
    default: return true;
    }
}

// A grid of Big tiles fills the chip in whole rounds of resident
// workgroups.  When its last round would be less than a fifth full, the
// rows of that round go to a second launch of Small tiles (a quarter of
// the work each, so about four times as many run at once); each output
// tile still accumulates all of K in block order, so the bits are
// unchanged.  (Measured: a last round that is fuller already runs faster
// than a full one, and the second launch's own gap and per-block latency
// then cost more than the split saves.)
template <class Big, class Small>
hipError_t launch_tail_split(const WeightView &w, const uint8_t *xq, int64_t row_bytes,
                             const uint16_t *xdT, int64_t ld_dx, int64_t M, float *y,
                             int64_t ldy, const EpiParams &epi, hipStream_t stream) {
    const int64_t n_tiles = (w.N + Big::BN - 1) / Big::BN;
    const int64_t m_tiles = (M + Big::BM - 1) / Big::BM;
    const int64_t T = m_tiles * n_tiles, S = resident_tiles<Big>();
    int64_t rows_main = M;
    if (S > 0 && T > S && T % S != 0 && 5 * (T % S) < S) {
        const int64_t m_main = (T / S) * S / n_tiles;  // whole Big row tiles in full rounds
        rows_main = m_main * Big::BM;
    }
    EpiParams tail;
    float *yt = y;
    if (rows_main >= M || !shift_rows(epi, rows_main, yt, ldy, tail))
        return dispatch<Big>(w, xq, xdT, ld_dx, M, y, ldy, epi, stream);
    hipError_t e = dispatch<Big>(w, xq, xdT, ld_dx, rows_main, y, ldy, epi, stream);
    if (e != hipSuccess) return e;
    return dispatch<Small>(w, xq + rows_main * row_bytes, xdT + rows_main, ld_dx, M - rows_main,
                           yt, ldy, tail, stream);
}

}  // namespace mmq16

hipError_t launch_mmq_f16(const WeightView &w, const _Float16 *xh, const uint16_t *xdT,
                          int64_t ld_dx, int64_t M, float *y, int64_t ldy,
                          const EpiParams &epi, hipStream_t stream) {
    if (M == 0 || w.N == 0) return hipSuccess;
    if (!w.qh || !mmq_args_ok(w, xh, xdT, ld_dx, M)) return hipErrorInvalidValue;
    using Big = mmq16::Cfg<128, 3, false, 1, true, false, 2>;
    using Small = mmq16::Cfg<64, 3, false, 1, true, false, 1>;
    return mmq16::launch_tail_split<Big, Small>(w, reinterpret_cast<const uint8_t *>(xh),
                                                w.K_pad * 2, xdT, ld_dx, M, y, ldy, epi, stream);
}

hipError_t launch_mmq_i8(const WeightView &w, const int8_t *xq, const uint16_t *xdT,
                         int64_t ld_dx, int64_t M, float *y, int64_t ldy, const EpiParams &epi,
                         hipStream_t stream) {
    if (M == 0 || w.N == 0) return hipSuccess;
    if (!w.qs || !mmq_args_ok(w, xq, xdT, ld_dx, M)) return hipErrorInvalidValue;
    // One launch: with three K blocks per stage a sparse last round of tiles
    // costs less than the second launch a tail split would add (fc1 at
    // M = 23,328: 368 against 377 us).
    using Big = mmq16::Cfg<128, 2, false, 1, true, true, 2, 3>;
    return mmq16::dispatch<Big>(w, xq, xdT, ld_dx, M, y, ldy, epi, stream);
}

}  // namespace s2x
