// s2x_attn.hip -- bidirectional multi-head attention for SigLIP2 (d_head 72)
// on gfx950 f16 MFMA, over packed variable-length segments.
//
// Staging (k_attn_prep) replaces the reference's QKV bias + split + pad +
// f16 cast (src/cuda/siglip2_megakernel.cu:160-267): from the QKV GEMM rows
// [q | k | v] (+ bias) it writes, per segment and head,
//   Q  [len_pad][d_pad]  f16   (d zero-padded 72 -> 80)
//   K  [len_pad][d_pad]  f16
//   Vt [dv_pad][len_pad] f16   (V transposed, d zero-padded 72 -> 96)
// (len_pad = segment length rounded up to 128)
// with every padding slot an exact zero.
//
// Flash attention (k_attn) computes S^T = K Q^T with v_mfma_f32_32x32x16_f16
// so that the result layout puts one query per lane (column l & 31) and 16
// keys per lane in registers: the online-softmax max / sum are lane-local
// plus one exchange with lane l ^ 32, and the P values are already in the
// B-operand layout of the next product O^T = V^T P^T, whose result again
// holds one query per lane -- no shuffles of P or of the output rescale.
//
// k-index convention for an f16 32x32x16 MFMA operand: lane l, slot s <-> k
// = 8*(s/4) + 4*(l/32) + s%4 for the P V product (the layout P has as an S^T
// result) and k = 8*(l/32) + s for Q K^T.  A and B use the same convention,
// so the contraction is complete whatever the hardware's own k order is.
#include "s2x_device.h"
#include "s2x_kernels.h"

#include <algorithm>
#include <type_traits>

namespace s2x {

static inline int64_t round_up(int64_t a, int64_t b) { return (a + b - 1) / b * b; }

AttnLayout attn_layout(int64_t n_seg, int64_t max_len, int64_t n_head, int64_t d_head) {
    AttnLayout L;
    L.n_seg = n_seg;
    L.max_len = max_len;
    L.n_head = n_head;
    L.d_head = d_head;
    L.d_pad = round_up(d_head, 16);
    L.dv_pad = round_up(d_head, 32);
    L.len_pad = round_up(max_len, 128);  // whole 128-query tiles stay in bounds
    const size_t qk = (size_t)(n_seg * n_head * L.len_pad * L.d_pad) * 2;
    const size_t vt = (size_t)(n_seg * n_head * L.dv_pad * L.len_pad) * 2;
    L.q_off = 0;
    L.k_off = round_up((int64_t)qk, 256);
    L.vt_off = L.k_off + round_up((int64_t)qk, 256);
    L.planes_bytes = L.vt_off + round_up((int64_t)vt, 256);
    // packed row -> (segment, position) table of the fused QKV entry point
    L.rowmap_off = L.planes_bytes;
    L.bytes = L.rowmap_off + round_up(n_seg * max_len * 4, 256);
    return L;
}


// ---------------------------------------------------------------------------
// staging: one workgroup per (64-position tile, head, segment)
// ---------------------------------------------------------------------------
constexpr int PREP_T = 64;

__global__ __launch_bounds__(256) void k_attn_prep(
    const float *__restrict__ qkv, int64_t ld, const float *__restrict__ bias,
    const int32_t *__restrict__ seg_start, const int32_t *__restrict__ seg_len, int n_head,
    int d_head, int d_pad, int dv_pad, int len_pad, _Float16 *__restrict__ Q,
    _Float16 *__restrict__ K, _Float16 *__restrict__ Vt) {
    __shared__ _Float16 vs[PREP_T][97];  // one tile of V, d <= 96
    const int tile = blockIdx.x, h = blockIdx.y, sg = blockIdx.z;
    const int p0 = tile * PREP_T;
    const int len = seg_len[sg];
    const int64_t row0 = seg_start[sg];
    const int H = n_head * d_head;
    const int64_t head_qk = ((int64_t)sg * n_head + h) * len_pad * d_pad;
    const int64_t head_vt = ((int64_t)sg * n_head + h) * dv_pad * len_pad;

    // Q and K rows: element (p, d) of the tile, d fastest
    for (int i = threadIdx.x; i < PREP_T * d_pad; i += blockDim.x) {
        const int p = i / d_pad, d = i % d_pad;
        const int pos = p0 + p;
        float q = 0.0f, k = 0.0f;
        if (pos < len && d < d_head) {
            const float *r = qkv + (row0 + pos) * ld + h * d_head + d;
            q = r[0] + bias[h * d_head + d];
            k = r[H] + bias[H + h * d_head + d];
        }
        Q[head_qk + (int64_t)pos * d_pad + d] = f32_to_f16(q);  // (mm + bias) in f32, then f16
        K[head_qk + (int64_t)pos * d_pad + d] = f32_to_f16(k);
    }
    // V tile into LDS (d fastest reads), then transposed out (p fastest writes)
    for (int i = threadIdx.x; i < PREP_T * dv_pad; i += blockDim.x) {
        const int p = i / dv_pad, d = i % dv_pad;
        const int pos = p0 + p;
        float v = 0.0f;
        if (pos < len && d < d_head)
            v = qkv[(row0 + pos) * ld + 2 * H + h * d_head + d] + bias[2 * H + h * d_head + d];
        vs[p][d] = f32_to_f16(v);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < PREP_T * dv_pad; i += blockDim.x) {
        const int d = i / PREP_T, p = i % PREP_T;
        Vt[head_vt + (int64_t)d * len_pad + p0 + p] = vs[p][d];
    }
}

// Every row starts as ROW_NONE (no segment covers it: the QKV epilogue
// stores nothing for it), then rowmap[seg_start[s] + pos] = s << 16 | pos
// for pos < min(seg_len[s], max_len); entries outside [0, n_rows) are
// skipped.  Both are kernels, so a captured encode replays them.
__global__ __launch_bounds__(256) void k_rowmap_clear(int32_t *__restrict__ rowmap, int64_t n_rows) {
    const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r < n_rows) rowmap[r] = ROW_NONE;
}

__global__ __launch_bounds__(256) void k_rowmap(const int32_t *__restrict__ seg_start,
                                                const int32_t *__restrict__ seg_len,
                                                int32_t *__restrict__ rowmap, int64_t n_rows) {
    const int sg = blockIdx.y;
    const int pos = blockIdx.x * 256 + threadIdx.x;
    const int64_t r = (int64_t)seg_start[sg] + pos;
    if (pos < seg_len[sg] && r >= 0 && r < n_rows) rowmap[r] = (sg << 16) | pos;
}

hipError_t launch_rowmap(const int32_t *seg_start, const int32_t *seg_len, int64_t n_seg,
                         int64_t max_len, int32_t *rowmap, int64_t n_rows, hipStream_t stream) {
    if (n_rows == 0) return hipSuccess;
    if (n_seg > 32767 || max_len > 65535 || n_rows > (int64_t)1 << 40) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_rowmap_clear, dim3((unsigned)((n_rows + 255) / 256)), dim3(256), 0, stream,
                       rowmap, n_rows);
    if (n_seg == 0 || max_len == 0) return hipGetLastError();
    hipLaunchKernelGGL(k_rowmap, dim3((unsigned)((max_len + 255) / 256), (unsigned)n_seg),
                       dim3(256), 0, stream, seg_start, seg_len, rowmap, n_rows);
    return hipGetLastError();
}

EpiParams epi_qkv(const AttnLayout &L, void *ws, const float *qkv_bias, const int32_t *rowmap) {
    uint8_t *base = reinterpret_cast<uint8_t *>(ws);
    EpiParams p{EPI_QKV, qkv_bias, nullptr, 0, 0, 0};
    p.q = reinterpret_cast<_Float16 *>(base + L.q_off);
    p.k = reinterpret_cast<_Float16 *>(base + L.k_off);
    p.vt = reinterpret_cast<_Float16 *>(base + L.vt_off);
    p.rowmap = rowmap;
    p.n_head = (int)L.n_head;
    p.d_head = (int)L.d_head;
    p.d_pad = (int)L.d_pad;
    p.dv_pad = (int)L.dv_pad;
    p.len_pad = (int)L.len_pad;
    return p;
}

hipError_t launch_attn_prep(const float *qkv, int64_t ld_qkv, const float *qkv_bias,
                            const int32_t *seg_start, const int32_t *seg_len,
                            const AttnLayout &L, void *ws, hipStream_t stream) {
    if (L.n_seg == 0) return hipSuccess;
    uint8_t *base = reinterpret_cast<uint8_t *>(ws);
    const dim3 grid((unsigned)(L.len_pad / PREP_T), (unsigned)L.n_head, (unsigned)L.n_seg);
    hipLaunchKernelGGL(k_attn_prep, grid, dim3(256), 0, stream, qkv, ld_qkv, qkv_bias,
                       seg_start, seg_len, (int)L.n_head, (int)L.d_head, (int)L.d_pad,
                       (int)L.dv_pad, (int)L.len_pad,
                       reinterpret_cast<_Float16 *>(base + L.q_off),
                       reinterpret_cast<_Float16 *>(base + L.k_off),
                       reinterpret_cast<_Float16 *>(base + L.vt_off));
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Q8_1 of the attention output, folded into the flash kernel for 72-wide
// heads in groups of four (288 columns = 9 blocks of 32): head r = h % 4
// owns whole blocks {0, 1}, {3}, {5}, {7, 8} of its group (r = 0 .. 3) and
// quantizes them in its epilogue; blocks 2, 4, 6 straddle heads (r, r + 1),
// so their columns are written as f32 and a second pass (k_quant_straddle)
// quantizes them -- or, where a workgroup runs all four heads of a group in
// turn (launches of enough workgroups, batch 32), each lane keeps its
// columns of the block the next head completes in LDS, and that head's
// epilogue quantizes it.  All apply k_quantize_q8_1's arithmetic to the same
// f32 values: the same bits as quantizing the whole f32 output.
// ---------------------------------------------------------------------------
// One Q8_1 block of a row from this lane's 16 values v[4 k + i] (columns
// 8 k + 4 lh + i of the block, k, i = 0..3) and lane l ^ 32's (the other
// 4 columns of each 8): quants at qblk + 8 k + 4 lh, its scale word at *ds.
__device__ __forceinline__ void q81_block16(const float (&v)[16], int lh, int8_t *qblk,
                                            uint32_t *ds) {
    float a = 0.0f;
#pragma unroll
    for (int t = 0; t < 16; ++t) a = fmaxf(a, fabsf(v[t]));
    a = fmaxf(a, __shfl_xor(a, 32));
    const float d = a / 127.0f;
    const float qinv = a != 0.0f ? 127.0f / a : 0.0f;
    int sq = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int q0 = q8_round(v[4 * k], qinv), q1 = q8_round(v[4 * k + 1], qinv);
        const int q2 = q8_round(v[4 * k + 2], qinv), q3 = q8_round(v[4 * k + 3], qinv);
        *reinterpret_cast<uint32_t *>(qblk + 8 * k + 4 * lh) = pack4_i8(q0, q1, q2, q3);
        sq += q0 + q1 + q2 + q3;
    }
    sq += __shfl_xor(sq, 32);
    if (lh == 0) *ds = (uint32_t)f32_to_f16_bits(d) | ((uint32_t)f32_to_f16_bits((float)sq * d) << 16);
}

template <int M0>  // first 8-column group of the block within the head
__device__ __forceinline__ void attn_q81_block(const v16f (&o)[3], float inv, int lh,
                                               int8_t *qrow, uint32_t *dsrow, int kb) {
    float v[16];
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i) v[4 * k + i] = o[(M0 + k) / 4][4 * ((M0 + k) % 4) + i] * inv;
    // lane lh holds columns 8 m + 4 lh + 0..3 of each group m: the block is
    // this lane's 16 values and lane l ^ 32's
    q81_block16(v, lh, qrow + 8 * M0, dsrow + kb);
}

template <int M>  // an 8-column group written as f32 (part of a straddling block)
__device__ __forceinline__ void attn_f32_group(const v16f (&o)[3], float inv, int lh, float *orow) {
    const float4 v = make_float4(o[M / 4][4 * (M % 4)] * inv, o[M / 4][4 * (M % 4) + 1] * inv,
                                 o[M / 4][4 * (M % 4) + 2] * inv, o[M / 4][4 * (M % 4) + 3] * inv);
    *reinterpret_cast<float4 *>(orow + 8 * M + 4 * lh) = v;
}

// Epilogue of one query row for head position R = h % 4 within its group.
template <int R>
__device__ __forceinline__ void attn_q81_row(const v16f (&o)[3], float inv, int lh, float *orow,
                                             int8_t *qrow, uint32_t *dsrow, int kb0) {
    if constexpr (R == 0) {
        attn_q81_block<0>(o, inv, lh, qrow, dsrow, kb0);
        attn_q81_block<4>(o, inv, lh, qrow, dsrow, kb0 + 1);
        attn_f32_group<8>(o, inv, lh, orow);
    } else if constexpr (R == 1) {
        attn_f32_group<0>(o, inv, lh, orow);
        attn_f32_group<1>(o, inv, lh, orow);
        attn_f32_group<2>(o, inv, lh, orow);
        attn_q81_block<3>(o, inv, lh, qrow, dsrow, kb0 + 3);
        attn_f32_group<7>(o, inv, lh, orow);
        attn_f32_group<8>(o, inv, lh, orow);
    } else if constexpr (R == 2) {
        attn_f32_group<0>(o, inv, lh, orow);
        attn_f32_group<1>(o, inv, lh, orow);
        attn_q81_block<2>(o, inv, lh, qrow, dsrow, kb0 + 5);
        attn_f32_group<6>(o, inv, lh, orow);
        attn_f32_group<7>(o, inv, lh, orow);
        attn_f32_group<8>(o, inv, lh, orow);
    } else {
        attn_f32_group<0>(o, inv, lh, orow);
        attn_q81_block<1>(o, inv, lh, qrow, dsrow, kb0 + 7);
        attn_q81_block<5>(o, inv, lh, qrow, dsrow, kb0 + 8);
    }
}

// Epilogue of one query row for head R of a group of four run by one
// workgroup: qg / dsg are the row's quants and scale words of the group
// (288 columns, blocks 0..8); st[64 i], i < 12, is this lane's LDS slot i,
// which carries the 8-column groups of head R - 1 that open block 2 R.
template <int R>
__device__ __forceinline__ void attn_q81_group_row(const v16f (&o)[3], float inv, int lh,
                                                   int8_t *qg, uint32_t *dsg, float *st) {
    constexpr int NK = R;        // 8-column groups of block 2 R held from head R - 1
    constexpr int NH = 4 - NK;   // its groups from this head: 0 .. NH - 1
    int8_t *qh = qg + 72 * R;    // this head's first column
    if constexpr (R > 0) {
        float v[16];
#pragma unroll
        for (int k = 0; k < NK; ++k)
#pragma unroll
            for (int i = 0; i < 4; ++i) v[4 * k + i] = st[64 * (4 * k + i)];
#pragma unroll
        for (int k = 0; k < NH; ++k)
#pragma unroll
            for (int i = 0; i < 4; ++i) v[4 * (NK + k) + i] = o[k / 4][4 * (k % 4) + i] * inv;
        q81_block16(v, lh, qg + 64 * R, dsg + 2 * R);
    }
    // whole blocks of this head, then the groups that open block 2 R + 2
    if constexpr (R == 0) {
        attn_q81_block<0>(o, inv, lh, qh, dsg, 0);
        attn_q81_block<4>(o, inv, lh, qh, dsg, 1);
    } else if constexpr (R == 1) {
        attn_q81_block<3>(o, inv, lh, qh, dsg, 3);
    } else if constexpr (R == 2) {
        attn_q81_block<2>(o, inv, lh, qh, dsg, 5);
    } else {
        attn_q81_block<1>(o, inv, lh, qh, dsg, 7);
        attn_q81_block<5>(o, inv, lh, qh, dsg, 8);
    }
    if constexpr (R < 3) {
        constexpr int NS = R + 1;  // groups 9 - NS .. 8 of this head
#pragma unroll
        for (int k = 0; k < NS; ++k)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                st[64 * (4 * k + i)] = o[(9 - NS + k) / 4][4 * ((9 - NS + k) % 4) + i] * inv;
    }
}

// The straddling blocks 9 g + 2, + 4, + 6 of every 288-column group, from the
// f32 rows: one 8-lane group per (row, block), as k_quantize_q8_1.
__global__ __launch_bounds__(256) void k_quant_straddle(const float *__restrict__ x, int64_t ldx,
                                                         int64_t M, int64_t n_grp, Q81Out o,
                                                         int64_t ld_q) {
    const int64_t g = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 3;
    const int sub = threadIdx.x & 7;
    const int64_t per_row = 3 * n_grp;
    if (g >= M * per_row) return;  // whole 8-lane groups leave together
    const int64_t m = g / per_row, i = g - m * per_row;
    const int64_t kb = 9 * (i / 3) + 2 + 2 * (i % 3);
    const int64_t c = kb * QK + sub * 4;
    const float4 t = *reinterpret_cast<const float4 *>(x + m * ldx + c);
    // from 0, as a running fmaxf: NaNs are passed over, a block of NaNs has amax 0
    float a = fmaxf(fmaxf(fmaxf(fabsf(t.x), fabsf(t.y)), fmaxf(fabsf(t.z), fabsf(t.w))), 0.0f);
    a = group8_max(a);
    const float d = a / 127.0f;
    const float inv = a != 0.0f ? 127.0f / a : 0.0f;
    const int q0 = q8_round(t.x, inv), q1 = q8_round(t.y, inv);
    const int q2 = q8_round(t.z, inv), q3 = q8_round(t.w, inv);
    *reinterpret_cast<uint32_t *>(o.qs + m * ld_q + c) = pack4_i8(q0, q1, q2, q3);
    const int s = group8_isum(q0 + q1 + q2 + q3);
    if (sub == 0)
        o.ds[m * o.ld_ds + kb] =
            (uint32_t)f32_to_f16_bits(d) | ((uint32_t)f32_to_f16_bits((float)s * d) << 16);
}

// ---------------------------------------------------------------------------
// flash attention: one workgroup = FA_WAVES waves x 32 queries of one
// (segment, head); 64-key tiles of K and V^T staged through LDS (double
// buffered).  12 waves: each thread stages one K and one V^T chunk per
// tile, which keeps the kernel at 151 VGPRs, i.e. 3 waves per SIMD -- one
// workgroup per CU, and 1,024 workgroups (4 full rounds) at 32 x 729.
// Specialised for d_pad = 80 (5 k-steps) and dv_pad = 96 (3 row tiles).
// ---------------------------------------------------------------------------
constexpr int FA_DP = 80;              // Q/K row length (halves)
constexpr int FA_DV = 96;              // V^T rows
constexpr int FA_KT = 64;              // keys per LDS tile
constexpr int FA_KP = FA_DP + 8;       // K tile pitch (halves): conflict-free 16-byte reads
constexpr int FA_VP = FA_KT + 8;       // V^T tile pitch (halves): 16-byte rows, conflict-free reads
constexpr int FA_ONES = 88;            // V^T padding row held at 1.0: O^T row 88 = sum of P
constexpr int FA_STAGE = FA_KT * FA_KP + FA_DV * FA_VP;  // halves per buffer
constexpr int FA_WAVES = 12;  // waves (32 queries each) per workgroup
constexpr int FA_WAVES_SMALL = 4;  // the same for launches of few workgroups
constexpr float P_SHIFT = 15.0f;  // log2 of the largest P of a row (<= 65504 as f16)

// G4 (with QUANT): one workgroup runs the four heads of a group in turn and
// quantizes every Q8_1 block of its rows itself (no f32 output, no second
// pass); each lane's columns of the block that the next head completes wait
// in an LDS slot of its own.
template <bool P_SPLIT, int NW, bool QUANT, bool G4 = false>
__global__ __launch_bounds__(64 * NW) void k_attn(
    const _Float16 *__restrict__ Q, const _Float16 *__restrict__ K,
    const _Float16 *__restrict__ Vt, const int32_t *__restrict__ seg_start,
    const int32_t *__restrict__ seg_len, const uint8_t *__restrict__ key_valid,
    int n_head, int d_head, int len_pad, int n_qt, float scale_log2, float *__restrict__ out,
    int64_t ld_out, Q81Out qo, int64_t ld_q) {
    static_assert(!G4 || QUANT, "the grouped form writes Q8_1 only");
    __shared__ __align__(16) _Float16 lds[2 * FA_STAGE];
    __shared__ float stash[G4 ? 12 * 64 * NW : 1];
    // (query tile, head or group of four heads, segment), query tile
    // fastest, in XCD-contiguous order: the query tiles of one head share
    // their XCD's L2 for K and V^T
    constexpr int HPW = G4 ? 4 : 1;  // heads per workgroup
    const int n_hg = n_head / HPW;
    const int wg = xcd_linear(blockIdx.x, gridDim.x);
    const int qt = wg % n_qt, hg = (wg / n_qt) % n_hg, sg = wg / (n_qt * n_hg);
    const int len = seg_len[sg];
    constexpr int NT = 64 * NW, QT = 32 * NW;  // threads, queries per workgroup
    if (qt * QT >= len) return;  // whole workgroup past the segment
    const int64_t row0 = seg_start[sg];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 31, lh = lane >> 5;
    // Q^T fragments (B operand): lane holds query q, d = 16 t + 8 lh + s
    const int q = qt * QT + wave * 32 + lr;
    const bool active = __builtin_amdgcn_readfirstlane(qt * QT + wave * 32) < len;
    // (a workgroup's last queries may lie past len_pad, a multiple of 128:
    // they read row len_pad - 1 and are never stored)
    const int qrow = min(q, len_pad - 1);

    // (every head ends with its last tile's barrier: the next head's first
    // LDS store cannot overtake a read of this one's)
    for (int hr = 0; hr < HPW; ++hr) {
        const int h = hg * HPW + hr;
        const int64_t head_qk = ((int64_t)sg * n_head + h) * len_pad * FA_DP;
        const int64_t head_vt = ((int64_t)sg * n_head + h) * FA_DV * len_pad;
        const _Float16 *Kh = K + head_qk;
        const _Float16 *Vh = Vt + head_vt;
        v8h qf[5];
#pragma unroll
        for (int t = 0; t < 5; ++t)
            qf[t] = *reinterpret_cast<const v8h *>(Q + head_qk + (int64_t)qrow * FA_DP + 16 * t + 8 * lh);

        v16f o[3];
#pragma unroll
        for (int j = 0; j < 3; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[j][r] = 0.0f;
        float m_run = -INFINITY, mc_run = -INFINITY;

        const int n_tiles = (len + FA_KT - 1) / FA_KT;

        // global -> registers for one key tile: K 64x80 halves (10240 B contiguous,
        // 640 chunks of 16 B), V^T 96 rows x 64 halves (128 B each, 768 chunks)
        constexpr int K_CH = FA_KT * FA_DP / 8, V_CH = FA_DV * FA_KT / 8;
        constexpr int KC = (K_CH + NT - 1) / NT, VC = (V_CH + NT - 1) / NT;
        struct Tile {
            uint4 k[KC], v[VC];
        };
        // threads past the last K chunk re-load it (always in bounds) and later
        // rewrite it with the value it already has
        int kc[KC];
#pragma unroll
        for (int i = 0; i < KC; ++i) kc[i] = min(tid + i * NT, K_CH - 1);
        // One code path for every tile (the edge masking happens at the LDS
        // store): the next tile's loads stay in flight through the current
        // tile's MFMAs, with no merge of differently loaded registers that would
        // make the compiler wait for them right after issue.
        auto gload = [&](int t) {
            const int k0 = t * FA_KT;
            const uint4 *ks = reinterpret_cast<const uint4 *>(Kh + (int64_t)k0 * FA_DP);
            Tile g;
#pragma unroll
            for (int i = 0; i < KC; ++i) g.k[i] = ks[kc[i]];
#pragma unroll
            for (int i = 0; i < VC; ++i) {
                const int c = tid + i * NT;  // V chunk c: row c/8, col (c%8)*8 halves
                if (V_CH % NT == 0 || c < V_CH)
                    g.v[i] = *reinterpret_cast<const uint4 *>(Vh + (int64_t)(c >> 3) * len_pad + k0 +
                                                              (c & 7) * 8);
            }
            return g;
        };
        auto sstore = [&](int buf, int t, const Tile &g) {
            _Float16 *kl = lds + buf * FA_STAGE;
            _Float16 *vl = kl + FA_KT * FA_KP;
            const auto kput = [&](int c, uint4 v) {
                *reinterpret_cast<uint4 *>(kl + (c / 10) * FA_KP + (c % 10) * 8) = v;
            };
#pragma unroll
            for (int i = 0; i < KC; ++i) kput(kc[i], g.k[i]);
            // V^T rows keep each 16-key group in the order [0-3, 8-11, 4-7,
            // 12-15]: the 8 keys a lane feeds to one PV MFMA (4 lh + 0..3 and
            // 8 + 4 lh + 0..3, the S^T result layout) are then one 16-byte read
            const auto vput = [&](int i, uint4 v) {
                const int c = tid + i * NT;
                const int row = c >> 3, ch = c & 7;
                // keys past the segment hold zeros or stale finite data; zero
                // them so a stale NaN/Inf can never meet a zero probability
                // (only the tile holding the segment end has such keys)
                const int valid = len - (t * FA_KT + ch * 8);
                if (valid < 8) {
                    const auto keep = [valid](int j) {
                        return (valid > 2 * j ? 0xffffu : 0u) | (valid > 2 * j + 1 ? 0xffff0000u : 0u);
                    };
                    v = make_uint4(v.x & keep(0), v.y & keep(1), v.z & keep(2), v.w & keep(3));
                }
                if (row == FA_ONES) v = make_uint4(0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u);
                _Float16 *base = vl + row * FA_VP + (ch >> 1) * 16 + (ch & 1) * 4;
                *reinterpret_cast<uint2 *>(base) = make_uint2(v.x, v.y);
                *reinterpret_cast<uint2 *>(base + 8) = make_uint2(v.z, v.w);
            };
#pragma unroll
            for (int i = 0; i < VC; ++i)
                if (V_CH % NT == 0 || tid + i * NT < V_CH) vput(i, g.v[i]);
        };

        const int n_plain = key_valid ? 0 : len / FA_KT;  // whole tiles without a key mask
        sstore(0, 0, gload(0));
        __syncthreads();

        // one 64-key tile; MASK: the tile holding the segment end, or a key mask
        auto tile = [&](int t, auto maskc) {
            constexpr bool MASK = decltype(maskc)::value;
            const int buf = t & 1;
            // (past the last tile: the last tile again, never stored)
            const Tile nxt = gload(min(t + 1, n_tiles - 1));
            const _Float16 *kl = lds + buf * FA_STAGE;
            const _Float16 *vl = kl + FA_KT * FA_KP;
            // a wave whose 32 queries all lie past the segment end only stages
            // tiles for the others
            if (active) {
            // S^T for the tile's two 32-key halves (raw q.k, unscaled)
            // (both halves' K fragments read up front, then the two
            // independent MFMA chains interleaved)
            v16f sc[2] = {};
            v8h kf[2][5];
#pragma unroll
            for (int st = 0; st < 5; ++st)
#pragma unroll
                for (int sub = 0; sub < 2; ++sub)
                    kf[sub][st] = *reinterpret_cast<const v8h *>(kl + (sub * 32 + lr) * FA_KP + 16 * st + 8 * lh);
#pragma unroll
            for (int st = 0; st < 5; ++st)
#pragma unroll
                for (int sub = 0; sub < 2; ++sub)
                    sc[sub] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[sub][st], qf[st], sc[sub], 0, 0, 0);
            // mask (only the tile holding the segment end, or a key mask), then
            // the tile max; one softmax rescale per 64 keys
            const int kbase = t * FA_KT;
            if constexpr (MASK) {
#pragma unroll
                for (int sub = 0; sub < 2; ++sub)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = kbase + sub * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                        bool ok = key < len;
                        if (key_valid) ok = ok && key_valid[row0 + min(key, len - 1)] != 0;
                        sc[sub][r] = ok ? sc[sub][r] : -INFINITY;
                    }
            }
            float mt = -INFINITY;
#pragma unroll
            for (int sub = 0; sub < 2; ++sub)
#pragma unroll
                for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sc[sub][r]);
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            // P = 2^(s scale_log2 - mc) with mc = m scale_log2 - P_SHIFT: the
            // largest P of a row is 2^P_SHIFT, not 1, so that the f16 pair below
            // keeps ~22 significant bits for P down to 2^-13 of the row maximum
            // (unshifted, the lo half turns f16-subnormal below 2^-4 and its
            // truncation biases every small P downward).  O and its P sum carry
            // the same factor, which cancels in O / sum.  alpha compares the two
            // exponent offsets actually used, so no rounding of mc enters it.
            const float m_new = fmaxf(m_run, mt);  // in raw score units (scale > 0)
            const float mc = m_new == -INFINITY ? 0.0f : fmaf(m_new, scale_log2, -P_SHIFT);
            const float alpha = __builtin_amdgcn_exp2f(mc_run - mc);  // 0 before the first key
            m_run = m_new;
            mc_run = m_new == -INFINITY ? -INFINITY : mc;
            // alpha is exactly 1 where the running max did not move: skip the
            // rescale when that holds for the whole wave (the common case once
            // the first tiles have set the max)
            if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
                for (int j = 0; j < 3; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[j][r] = o[j][r] * alpha;
            }
#pragma unroll
            for (int sub = 0; sub < 2; ++sub) {
                // P as f16 for the PV product; with P_SPLIT as a pair p ~ hi + lo
                // (hi = f16(p) rounded toward zero, lo = f16(p - hi) with p - hi
                // exact in f32): ~22 significant bits instead of 11.  Pairs of
                // values convert in one v_cvt_pkrtz_f16_f32, whose packed words
                // are the MFMA operand registers as they stand.
                float pv[16];
#pragma unroll
                for (int r = 0; r < 16; ++r) pv[r] = __builtin_amdgcn_exp2f(fmaf(sc[sub][r], scale_log2, -mc));
                uint32_t hw[8], lw[8];
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    const auto h2 = __builtin_amdgcn_cvt_pkrtz(pv[r], pv[r + 1]);
                    hw[r / 2] = __builtin_bit_cast(uint32_t, h2);
                    if (P_SPLIT) {
                        // p - hi in one v_fma_mix_f32 each (hi read as f16 from its
                        // half of the packed word, -1.0 as f32, p as f32): exact
                        float l0, l1;
                        asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]"
                            : "=v"(l0) : "v"(hw[r / 2]), "v"(pv[r]));
                        asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
                            : "=v"(l1) : "v"(hw[r / 2]), "v"(pv[r + 1]));
                        lw[r / 2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(l0, l1));
                    }
                }
                const v8h ph0 = __builtin_bit_cast(v8h, v4u{hw[0], hw[1], hw[2], hw[3]});
                const v8h ph1 = __builtin_bit_cast(v8h, v4u{hw[4], hw[5], hw[6], hw[7]});
                v8h pl0 = {}, pl1 = {};
                if (P_SPLIT) {
                    pl0 = __builtin_bit_cast(v8h, v4u{lw[0], lw[1], lw[2], lw[3]});
                    pl1 = __builtin_bit_cast(v8h, v4u{lw[4], lw[5], lw[6], lw[7]});
                }
                // O^T += V^T P^T (row FA_ONES of V^T is 1: O^T row FA_ONES sums P).
                // Each o[j] takes its products in the order hh 0 (hi, lo), hh 1
                // (hi, lo); consecutive MFMAs go to different j (independent).
                v8h vf[3][2];
#pragma unroll
                for (int j = 0; j < 3; ++j)
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
                        vf[j][hh] = *reinterpret_cast<const v8h *>(vl + (j * 32 + lr) * FA_VP + sub * 32 + 16 * hh + 8 * lh);
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
                    for (int j = 0; j < 3; ++j)
                        o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[j][hh], hh ? ph1 : ph0, o[j], 0, 0, 0);
                    if (P_SPLIT) {
#pragma unroll
                        for (int j = 0; j < 3; ++j)
                            o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[j][hh], hh ? pl1 : pl0, o[j], 0, 0, 0);
                    }
                }
            }
            }
            if (t + 1 < n_tiles) sstore(buf ^ 1, t + 1, nxt);
            __syncthreads();
        };
        // whole tiles without a key mask take the unmasked instance
        for (int t = 0; t < n_plain; ++t) tile(t, std::false_type{});
        for (int t = n_plain; t < n_tiles; ++t) tile(t, std::true_type{});

        // sum of P: O^T row FA_ONES = 64 + 24 (register 12 of lanes 0..31)
        static_assert(FA_ONES == 2 * 32 + 8 * 3 && FA_ONES >= FA_DP && FA_ONES < FA_DV, "ones row");
        const float l_tot = __shfl(o[2][12], lr);
        const float inv = 1.0f / l_tot;
        if (QUANT) {
            // (d_head 72, heads in groups of four: checked by the launcher)
            if (q < len) {
                const int64_t row = row0 + q;
                float *orow = out + row * ld_out + h * d_head;
                int8_t *qrow = qo.qs + row * ld_q + h * d_head;
                uint32_t *dsrow = qo.ds + row * qo.ld_ds;
                const int kb0 = 9 * (h >> 2);
                if constexpr (G4) {
                    int8_t *qg = qrow - 72 * hr;  // the group's first column
                    uint32_t *dsg = dsrow + kb0;
                    float *st = stash + wave * 64 * 12 + lane;
                    switch (hr) {
                    case 0: attn_q81_group_row<0>(o, inv, lh, qg, dsg, st); break;
                    case 1: attn_q81_group_row<1>(o, inv, lh, qg, dsg, st); break;
                    case 2: attn_q81_group_row<2>(o, inv, lh, qg, dsg, st); break;
                    default: attn_q81_group_row<3>(o, inv, lh, qg, dsg, st); break;
                    }
                } else {
                    switch (h & 3) {
                    case 0: attn_q81_row<0>(o, inv, lh, orow, qrow, dsrow, kb0); break;
                    case 1: attn_q81_row<1>(o, inv, lh, orow, qrow, dsrow, kb0); break;
                    case 2: attn_q81_row<2>(o, inv, lh, orow, qrow, dsrow, kb0); break;
                    default: attn_q81_row<3>(o, inv, lh, orow, qrow, dsrow, kb0); break;
                    }
                }
            }
        } else if (q < len) {
            float *orow = out + (row0 + q) * ld_out + h * d_head;
#pragma unroll
            for (int j = 0; j < 3; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d = j * 32 + 8 * g + 4 * lh;
                    if (d < d_head) {
                        const float4 v = make_float4(o[j][4 * g] * inv, o[j][4 * g + 1] * inv,
                                                     o[j][4 * g + 2] * inv, o[j][4 * g + 3] * inv);
                        *reinterpret_cast<float4 *>(orow + d) = v;
                    }
                }
        }
    }
}

hipError_t launch_attn(const void *ws, const int32_t *seg_start, const int32_t *seg_len,
                       const uint8_t *key_valid, const AttnLayout &L, float scale,
                       float *out, int64_t ld_out, hipStream_t stream, const Q81Out *qo,
                       int64_t n_rows) {
    if (L.n_seg == 0) return hipSuccess;
    if (L.d_pad != FA_DP || L.dv_pad != FA_DV || (L.d_head % 4) != 0) return hipErrorInvalidValue;
    const int64_t H = L.n_head * L.d_head;
    if (qo && (!attn_q81_fusable(L.n_head, L.d_head) || !qo->qs || !qo->ds || n_rows <= 0 ||
               qo->ld_ds < H / QK || ld_out < H || ld_out % 4 != 0))
        return hipErrorInvalidValue;
    const uint8_t *base = reinterpret_cast<const uint8_t *>(ws);
    const float log2e = 1.4426950408889634f;
    // 12-wave workgroups fill the chip from 256 of them up (batch 32: 1,024);
    // below that, 4-wave ones spread the same waves over 3x the CUs (batch
    // 1: 96 workgroups instead of 32).  Each query's arithmetic is the same.
    int NW = FA_WAVES;
    if (((L.max_len + 32 * NW - 1) / (32 * NW)) * L.n_head * L.n_seg < 256) NW = FA_WAVES_SMALL;
    const int64_t n_qt = (L.max_len + 32 * NW - 1) / (32 * NW);
    const bool qz = qo != nullptr;
    // with the Q8_1 output, 12-wave workgroups that each run a group of four
    // heads where those still number 256 or more (batch 32: 256, one per CU,
    // the same waves per CU as 1,024 one-head workgroups): no second pass
    const bool g4 = qz && NW == FA_WAVES && n_qt * (L.n_head / 4) * L.n_seg >= 256;
    const int64_t n_wg = n_qt * (g4 ? L.n_head / 4 : L.n_head) * L.n_seg;
    if (n_wg > 0x7fffffff) return hipErrorInvalidValue;
    using KFn = void (*)(const _Float16 *, const _Float16 *, const _Float16 *, const int32_t *,
                         const int32_t *, const uint8_t *, int, int, int, int, float, float *,
                         int64_t, Q81Out, int64_t);
    KFn kern;
    if (g4)
        kern = L.p_split ? k_attn<true, FA_WAVES, true, true> : k_attn<false, FA_WAVES, true, true>;
    else if (NW == FA_WAVES)
        kern = L.p_split ? (qz ? k_attn<true, FA_WAVES, true> : k_attn<true, FA_WAVES, false>)
                         : (qz ? k_attn<false, FA_WAVES, true> : k_attn<false, FA_WAVES, false>);
    else
        kern = L.p_split ? (qz ? k_attn<true, FA_WAVES_SMALL, true> : k_attn<true, FA_WAVES_SMALL, false>)
                         : (qz ? k_attn<false, FA_WAVES_SMALL, true> : k_attn<false, FA_WAVES_SMALL, false>);
    const Q81Out q_none{};
    hipLaunchKernelGGL(kern, dim3((unsigned)n_wg), dim3(64 * NW), 0, stream,
                       reinterpret_cast<const _Float16 *>(base + L.q_off),
                       reinterpret_cast<const _Float16 *>(base + L.k_off),
                       reinterpret_cast<const _Float16 *>(base + L.vt_off), seg_start, seg_len,
                       key_valid, (int)L.n_head, (int)L.d_head, (int)L.len_pad, (int)n_qt,
                       scale * log2e, out, ld_out, qz ? *qo : q_none, H);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !qz || g4) return e;
    // the blocks that straddle two heads, from the f32 columns just written
    // (rows of the packed segments: 0 .. n_rows - 1, every row a segment's)
    const int64_t groups = n_rows * 3 * (L.n_head / 4);
    hipLaunchKernelGGL(k_quant_straddle, dim3((unsigned)((groups * 8 + 255) / 256)), dim3(256), 0,
                       stream, out, ld_out, n_rows, L.n_head / 4, *qo, H);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// fp64 attention for short sequences (the text tower: 64 tokens).  Straight
// from the QKV GEMM rows: q/k/v = f16(f32(mm + bias)) as the reference casts
// them, then in double and in a fixed order -- score s_j = (sum_d q_d k_jd)
// * scale, max over valid keys, p_j = exp(s_j - max), den = sum_j p_j,
// acc_d = sum_j p_j v_jd (j ascending), out = f32(acc_d / den).  All but
// exp() round identically on any IEEE machine summing in the same order.
// One workgroup = one wave = 64 queries of one (segment, head); 64-key
// tiles of K and V staged in LDS as floats holding the f16 values.
// ---------------------------------------------------------------------------
constexpr int A64_T = 64;
constexpr int A64_DMAX = 80;

__global__ __launch_bounds__(64) void k_attn_f64(
    const float *__restrict__ qkv, int64_t ld, const float *__restrict__ bias,
    const int32_t *__restrict__ seg_start, const int32_t *__restrict__ seg_len,
    const uint8_t *__restrict__ key_valid, int n_head, int d_head, double scale,
    float *__restrict__ out, int64_t ld_out) {
    __shared__ float qs[A64_T][A64_DMAX + 1];
    __shared__ float ks[A64_T][A64_DMAX];
    __shared__ float vs[A64_T][A64_DMAX];
    const int qb = blockIdx.x, h = blockIdx.y, sg = blockIdx.z;
    const int len = seg_len[sg];
    if (qb * A64_T >= len) return;
    const int64_t row0 = seg_start[sg];
    const int H = n_head * d_head;
    const int lane = threadIdx.x;
    const int q = qb * A64_T + lane;
    auto f16r = [](float x) { return (float)f32_to_f16(x); };
    for (int i = lane; i < A64_T * d_head; i += A64_T) {
        const int p = i / d_head, d = i % d_head;
        const int pos = qb * A64_T + p;
        qs[p][d] = pos < len ? f16r(qkv[(row0 + pos) * ld + h * d_head + d] + bias[h * d_head + d]) : 0.0f;
    }
    const bool active = q < len;
    const int n_tiles = (len + A64_T - 1) / A64_T;
    auto load_kv = [&](int t) {
        __syncthreads();
        for (int i = lane; i < A64_T * d_head; i += A64_T) {
            const int p = i / d_head, d = i % d_head;
            const int pos = t * A64_T + p;
            float k = 0.0f, v = 0.0f;
            if (pos < len) {
                const float *r = qkv + (row0 + pos) * ld + h * d_head + d;
                k = f16r(r[H] + bias[H + h * d_head + d]);
                v = f16r(r[2 * H] + bias[2 * H + h * d_head + d]);
            }
            ks[p][d] = k;
            vs[p][d] = v;
        }
        __syncthreads();
    };
    auto score = [&](int j) {  // j local to the tile
        double acc = 0.0;
        for (int d = 0; d < d_head; ++d) acc = acc + (double)qs[lane][d] * (double)ks[j][d];
        return acc * scale;
    };
    auto valid = [&](int key) {
        return key < len && (key_valid == nullptr || key_valid[row0 + key] != 0);
    };
    // pass 1: max over valid keys
    double mx = -INFINITY;
    for (int t = 0; t < n_tiles; ++t) {
        load_kv(t);
        if (active)
            for (int j = 0; j < A64_T; ++j)
                if (valid(t * A64_T + j)) mx = fmax(mx, score(j));
    }
    // pass 2: exp, sum, PV
    double acc[A64_DMAX];
    for (int d = 0; d < A64_DMAX; ++d) acc[d] = 0.0;
    double den = 0.0;
    for (int t = 0; t < n_tiles; ++t) {
        load_kv(t);
        if (!active) continue;
        for (int j = 0; j < A64_T; ++j) {
            const int key = t * A64_T + j;
            if (key >= len) break;
            if (!valid(key)) continue;
            const double p = exp(score(j) - mx);
            den = den + p;
#pragma unroll
            for (int d = 0; d < A64_DMAX; ++d)
                if (d < d_head) acc[d] = acc[d] + p * (double)vs[j][d];
        }
    }
    if (active) {
        float *orow = out + (row0 + q) * ld_out + h * d_head;
#pragma unroll
        for (int d = 0; d < A64_DMAX; ++d)
            if (d < d_head) orow[d] = (float)(acc[d] / den);
    }
}

// The same arithmetic for segments of at most 64 tokens (the text prompts),
// spread over a workgroup of 1,024 lanes per (head, segment) instead of one
// lane per query: each score, each query's maximum, sum and each output
// element keeps its own sequential order (the keys ascending, d ascending),
// so the results are the bits of k_attn_f64; only independent sums run side
// by side.  Q, K, V are staged as the doubles of their f16 values (rows of
// 73 doubles: consecutive rows start 146 dwords apart, so a wave reading one
// d of 64 rows touches distinct banks), the scores and then the
// probabilities as doubles, all in dynamic LDS; no conversion in the inner
// loops, and a thread tests each probability against zero once for all of
// its output columns.  Launches of few (head, segment) pairs (the text
// batch: 80) split each pair's queries over up to 4 workgroups (gridDim.z),
// every one staging the whole segment: the work is fp64 arithmetic and LDS
// reads per query, and one workgroup per pair leaves most CUs idle.
constexpr int A64S_P = 73;
constexpr int A64S_LDS = (3 * A64_T * A64S_P + A64_T * (A64_T + 1) + 2 * A64_T) * 8;
constexpr int A64S_NT = 1024;                // threads per workgroup
constexpr int A64S_C = (A64S_P - 1 + 15) / 16;  // PV columns per thread (d_head <= 72)

__global__ __launch_bounds__(A64S_NT) void k_attn_f64_short(
    const float *__restrict__ qkv, int64_t ld, const float *__restrict__ bias,
    const int32_t *__restrict__ seg_start, const int32_t *__restrict__ seg_len,
    const uint8_t *__restrict__ key_valid, int n_head, int d_head, double scale,
    float *__restrict__ out, int64_t ld_out) {
    extern __shared__ __align__(16) double a64s[];
    double(*qs)[A64S_P] = reinterpret_cast<double(*)[A64S_P]>(a64s);
    double(*ks)[A64S_P] = qs + A64_T;
    double(*vs)[A64S_P] = ks + A64_T;
    double(*S)[A64_T + 1] = reinterpret_cast<double(*)[A64_T + 1]>(vs + A64_T);
    double *mx_s = &S[A64_T][0], *den_s = mx_s + A64_T;
    const int h = blockIdx.x, sg = blockIdx.y;
    const int len = seg_len[sg];
    // this workgroup's queries: [qa, qb) of the segment
    const int q_per = (len + (int)gridDim.z - 1) / (int)gridDim.z;
    const int qa = (int)blockIdx.z * q_per, qb = min(len, qa + q_per);
    if (qa >= qb) return;  // whole workgroup: nothing to write
    const int64_t row0 = seg_start[sg];
    const int H = n_head * d_head;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // staging: thread t takes column t % d_head of rows t / d_head + s k
    // (s = A64S_NT / d_head row groups); every load is issued up front and
    // unconditionally (rows past the segment read its last row, then store
    // zeros)
    {
        const int s_rows = A64S_NT / d_head;
        if (tid < s_rows * d_head) {
            const int d = tid % d_head, p0 = tid / d_head;
            const float bq = bias[h * d_head + d], bk = bias[H + h * d_head + d];
            const float bv = bias[2 * H + h * d_head + d];
            const float *col = qkv + row0 * ld + h * d_head + d;
            constexpr int NR = (A64_T + A64S_NT / 72 - 1) / (A64S_NT / 72);  // rows per thread
            float q[NR], k[NR], v[NR];
#pragma unroll
            for (int u = 0; u < NR; ++u) {
                const float *r = col + (int64_t)min(p0 + u * s_rows, len - 1) * ld;
                q[u] = r[0];
                k[u] = r[H];
                v[u] = r[2 * H];
            }
#pragma unroll
            for (int u = 0; u < NR; ++u) {
                const int p = p0 + u * s_rows;
                if (p < A64_T) {
                    const bool in = p < len;
                    qs[p][d] = in ? (double)(float)f32_to_f16(q[u] + bq) : 0.0;
                    ks[p][d] = in ? (double)(float)f32_to_f16(k[u] + bk) : 0.0;
                    vs[p][d] = in ? (double)(float)f32_to_f16(v[u] + bv) : 0.0;
                }
            }
        }
    }
    __syncthreads();
    // scores: wave w takes queries qa + w + 16 u (u < 4), lane j the key j:
    // four independent sums (each in d order) share one read of the key's row
    const bool key_ok = lane < len && (key_valid == nullptr || key_valid[row0 + lane] != 0);
    static_assert(A64S_NT / 64 * 4 == A64_T, "one query group per wave");
    if (qa + wave < qb) {
        // U = the wave's queries in range (1 .. 4), a template value so that
        // no sum is computed for a query of another workgroup
        const auto scores = [&](auto uc) {
            constexpr int U = decltype(uc)::value;
            double acc[U];
            int qi[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                acc[u] = 0.0;
                qi[u] = qa + wave + 16 * u;
            }
#pragma unroll 8
            for (int d = 0; d < d_head; ++d) {
                const double k = ks[lane][d];
#pragma unroll
                for (int u = 0; u < U; ++u) acc[u] = acc[u] + qs[qi[u]][d] * k;
            }
#pragma unroll
            for (int u = 0; u < U; ++u) S[qi[u]][lane] = key_ok ? acc[u] * scale : -INFINITY;
        };
        const int n_u = (qb - qa - wave + 15) / 16;
        if (n_u >= 4)
            scores(std::integral_constant<int, 4>{});
        else if (n_u == 3)
            scores(std::integral_constant<int, 3>{});
        else if (n_u == 2)
            scores(std::integral_constant<int, 2>{});
        else
            scores(std::integral_constant<int, 1>{});
    }
    __syncthreads();
    if (tid >= qa && tid < qb) {
        double m = -INFINITY;
        for (int j = 0; j < len; ++j) m = fmax(m, S[tid][j]);
        mx_s[tid] = m;
    }
    __syncthreads();
    for (int i = tid; i < (qb - qa) * A64_T; i += A64S_NT) {
        const int q = qa + (i >> 6), j = i & 63;
        if (j < len) {
            const double sc = S[q][j];
            S[q][j] = sc == -INFINITY ? 0.0 : exp(sc - mx_s[q]);
        }
    }
    __syncthreads();
    if (tid >= qa && tid < qb) {
        double den = 0.0;
        for (int j = 0; j < len; ++j) den = den + S[tid][j];
        den_s[tid] = den;
    }
    __syncthreads();
    // PV: thread t takes query qa + t / 16 and the columns d = t % 16 + 16 c,
    // so a probability read once serves A64S_C outputs
    {
        const int q = qa + (tid >> 4), d0 = tid & 15;
        double acc[A64S_C];
#pragma unroll
        for (int c = 0; c < A64S_C; ++c) acc[c] = 0.0;
        if (q < qb) {
#pragma unroll 2
            for (int j = 0; j < len; ++j) {
                const double p = S[q][j];
                // the row's values first (one wait for all of them); columns
                // d_head .. are padding or the next row: computed, not stored
                double vv[A64S_C];
#pragma unroll
                for (int c = 0; c < A64S_C; ++c) vv[c] = vs[j][d0 + 16 * c];
                if (p != 0.0) {
#pragma unroll
                    for (int c = 0; c < A64S_C; ++c) acc[c] = acc[c] + p * vv[c];
                }
            }
            float *orow = out + (row0 + q) * ld_out + h * d_head;
#pragma unroll
            for (int c = 0; c < A64S_C; ++c) {
                const int d = d0 + 16 * c;
                if (d < d_head) orow[d] = (float)(acc[c] / den_s[q]);
            }
        }
    }
}

hipError_t launch_attn_f64(const float *qkv, int64_t ld_qkv, const float *qkv_bias,
                           const int32_t *seg_start, const int32_t *seg_len,
                           const uint8_t *key_valid, int64_t n_seg, int64_t max_len,
                           int64_t n_head, int64_t d_head, float scale, float *out,
                           int64_t ld_out, hipStream_t stream) {
    if (n_seg == 0) return hipSuccess;
    if (d_head > A64_DMAX) return hipErrorInvalidValue;
    if (max_len <= A64_T && d_head < A64S_P) {
        static bool attr_set = false;  // idempotent; a racing second call repeats it
        if (!attr_set) {
            const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(k_attn_f64_short),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     A64S_LDS);
            if (e != hipSuccess) return e;
            attr_set = true;
        }
        // queries split over up to 4 workgroups while the pairs number
        // fewer than 256 (5 prompts x 16 heads: 3 each, 240 workgroups)
        const int64_t pairs = n_head * n_seg;
        const unsigned qsplit = (unsigned)std::max<int64_t>(1, std::min<int64_t>(4, 256 / pairs));
        hipLaunchKernelGGL(k_attn_f64_short, dim3((unsigned)n_head, (unsigned)n_seg, qsplit),
                           dim3(A64S_NT), A64S_LDS, stream, qkv, ld_qkv, qkv_bias, seg_start, seg_len, key_valid, (int)n_head,
                           (int)d_head, (double)scale, out, ld_out);
        return hipGetLastError();
    }
    const dim3 grid((unsigned)((max_len + A64_T - 1) / A64_T), (unsigned)n_head, (unsigned)n_seg);
    hipLaunchKernelGGL(k_attn_f64, grid, dim3(A64_T), 0, stream, qkv, ld_qkv, qkv_bias, seg_start,
                       seg_len, key_valid, (int)n_head, (int)d_head, (double)scale, out, ld_out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// single-query attention for the MAP probe head (src/siglip2_vision.cpp:
// 249-295): the probe query against one segment's keys, Q, K and V rounded to
// f16 as the reference's FA inputs are.  One workgroup of 1,024 threads per
// (head, segment): a key per thread for the scores (729 keys: one pass), the
// max and the sum reduced per wave and then over the 16 waves, and the PV
// product over 56 key groups x 18 four-column chunks (d_head 72), the groups'
// partial sums added in group order.  At batch 1 the 16 workgroups are the
// whole launch, so the work per thread, not the thread count, sets its time.
// ---------------------------------------------------------------------------
constexpr int A1_MAXLEN = (int)MAX_SEG_LEN;
constexpr int A1_NT = 1024;                     // threads per workgroup
constexpr int A1_NW = A1_NT / 64;               // waves per workgroup
constexpr int A1_GROUPS = A1_NT / 18;           // key groups of the PV pass (d_head 72)

// DH: d_head when known at compile time (the model's 72: the key row's
// loads all issued before its fmas), 0 for any other (runtime d_head).
template <int DH>
__global__ __launch_bounds__(A1_NT) void k_attn_1q(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    int64_t ld, const int32_t *__restrict__ seg_start, const int32_t *__restrict__ seg_len,
    int n_head, int d_head_rt, float scale, float *__restrict__ out) {
    const int d_head = DH ? DH : d_head_rt;
    __shared__ float p[A1_MAXLEN];
    __shared__ float red[A1_NW];
    __shared__ float part[A1_GROUPS][128];
    __shared__ float qf[128];
    const int h = blockIdx.x, sg = blockIdx.y;
    const int tid = threadIdx.x, wave = tid >> 6;
    const int len = seg_len[sg];
    const int64_t row0 = seg_start[sg];
    const int H = n_head * d_head;
    const float *qh = q + h * d_head;
    if (tid < d_head) qf[tid] = (float)f32_to_f16(qh[tid]);
    __syncthreads();
    // one key per thread; with d_head % 4 == 0 and 16-byte aligned rows the
    // row is read as float4 (same fma order over d)
    const bool v4 = (d_head % 4 == 0) && (ld % 4 == 0) &&
                    ((reinterpret_cast<uintptr_t>(k) & 15) == 0);
    float mx = -INFINITY;
    for (int j = tid; j < len; j += A1_NT) {
        // q is read from LDS in each pass (a broadcast read): hoisted out of
        // the loop into registers beside the key row it exceeded the 128
        // registers of a 1,024-thread workgroup and went to scratch memory,
        // reloaded in the loop (the 729-key batch-1 launch 15.8 -> 11.2 us
        // with this, same bits)
        asm volatile("" ::: "memory");
        const float *kr = k + (row0 + j) * ld + h * d_head;
        float acc = 0.0f;
        if constexpr (DH != 0) {
            float4 t[DH / 4];
#pragma unroll
            for (int i = 0; i < DH / 4; ++i) t[i] = *reinterpret_cast<const float4 *>(kr + 4 * i);
#pragma unroll
            for (int i = 0; i < DH / 4; ++i) {
                acc = fmaf(qf[4 * i], (float)f32_to_f16(t[i].x), acc);
                acc = fmaf(qf[4 * i + 1], (float)f32_to_f16(t[i].y), acc);
                acc = fmaf(qf[4 * i + 2], (float)f32_to_f16(t[i].z), acc);
                acc = fmaf(qf[4 * i + 3], (float)f32_to_f16(t[i].w), acc);
            }
        } else if (v4) {
            for (int d = 0; d < d_head; d += 4) {
                const float4 t = *reinterpret_cast<const float4 *>(kr + d);
                acc = fmaf(qf[d], (float)f32_to_f16(t.x), acc);
                acc = fmaf(qf[d + 1], (float)f32_to_f16(t.y), acc);
                acc = fmaf(qf[d + 2], (float)f32_to_f16(t.z), acc);
                acc = fmaf(qf[d + 3], (float)f32_to_f16(t.w), acc);
            }
        } else {
            for (int d = 0; d < d_head; ++d) acc = fmaf(qf[d], (float)f32_to_f16(kr[d]), acc);
        }
        const float s = acc * scale;
        p[j] = s;
        mx = fmaxf(mx, s);
    }
    mx = group_max<64>(mx);
    if ((tid & 63) == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < A1_NW; ++w) mx = fmaxf(mx, red[w]);
    float sum = 0.0f;
    for (int j = tid; j < len; j += A1_NT) {
        const float e = expf(p[j] - mx);
        p[j] = e;
        sum += e;
    }
    sum = group_sum<64>(sum);
    __syncthreads();  // every wave has read red[] (the max) before it is reused
    if ((tid & 63) == 0) red[wave] = sum;
    __syncthreads();  // ... and the p[] writes are visible to the PV pass
    float den = red[0];
#pragma unroll
    for (int w = 1; w < A1_NW; ++w) den = den + red[w];
    // out[d] = sum_j p_j v[j][d] / den: threads = key groups x 4-column
    // chunks of the head, each group's partial sums then added in group order
    const int nch = (d_head + 3) / 4;
    const int ng = min(A1_NT / nch, A1_GROUPS);
    const int grp = tid / nch, ch = tid - grp * nch;
    if (grp < ng) {
        float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const float *vh = v + h * d_head + 4 * ch;
        if (v4 && (reinterpret_cast<uintptr_t>(v) & 15) == 0) {
            // (unrolled: several rows' loads in flight; each a[i] still
            // takes its keys in order)
#pragma unroll 8
            for (int j = grp; j < len; j += ng) {
                const float4 t = *reinterpret_cast<const float4 *>(vh + (row0 + j) * ld);
                const float pj = p[j];
                a[0] = fmaf(pj, (float)(_Float16)t.x, a[0]);
                a[1] = fmaf(pj, (float)(_Float16)t.y, a[1]);
                a[2] = fmaf(pj, (float)(_Float16)t.z, a[2]);
                a[3] = fmaf(pj, (float)(_Float16)t.w, a[3]);
            }
        } else {
            for (int j = grp; j < len; j += ng) {
                const float *vr = vh + (row0 + j) * ld;
                const float pj = p[j];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (4 * ch + i < d_head) a[i] = fmaf(pj, (float)(_Float16)vr[i], a[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (4 * ch + i < d_head) part[grp][4 * ch + i] = a[i];
    }
    __syncthreads();
    if (tid < d_head) {
        float acc = part[0][tid];
        for (int g = 1; g < ng; ++g) acc = acc + part[g][tid];
        out[(int64_t)sg * H + h * d_head + tid] = acc / den;
    }
}

hipError_t launch_attn_1q(const float *q, const float *k, const float *v, int64_t ld,
                          const int32_t *seg_start, const int32_t *seg_len, int64_t n_seg,
                          int64_t n_head, int64_t d_head, float scale, float *out,
                          hipStream_t stream) {
    if (n_seg == 0) return hipSuccess;
    if (d_head > 128) return hipErrorInvalidValue;  // the PV partial sums hold 128 dims
    const bool dh72 = d_head == 72 && ld % 4 == 0 && (reinterpret_cast<uintptr_t>(k) & 15) == 0;
    hipLaunchKernelGGL(dh72 ? k_attn_1q<72> : k_attn_1q<0>, dim3((unsigned)n_head, (unsigned)n_seg), dim3(A1_NT), 0, stream,
                       q, k, v, ld, seg_start, seg_len, (int)n_head, (int)d_head, scale, out);
    return hipGetLastError();
}

}  // namespace s2x
