// k_gemm.hip -- prefill GEMM (m > 8) on int8 MFMA for gfx950.
//
// Replaces the M-row loop of candle-core 0.8.4 k_quants::matmul<T> at
// prefill (native/arm_ai_nif/src/llama_candle.rs:93, forward(&x[1,L], 0)):
// y[m][n] = sum over super-blocks b of the Q4_K . Q8_K block dot product
//   d_x[m,b] * (d_w[n,b] * S[m,n,b] - dmin_w[n,b] * Smin[m,n,b]),
//   S    = sum_j sc[n,b,j] * sum_{e in sub-block j} q[n,e] * qx[m,e]
//   Smin = sum_g bsums[m,b,g] * mn[n,b,g/2]
// with S and Smin exact integers, as in candle's vec_dot.
//
// Exactness on int8 MFMA.  sc*q reaches 63*15 = 945 and does not fit an
// int8 operand, so the 6-bit scale is split into two 3-bit digits,
// sc = 8*s1 + s0, and the weight operand becomes two int8 planes s1*q and
// s0*q (each <= 105).  Two v_mfma_i32_32x32x32_i8 per 32-element sub-block
// accumulate acc1 = sum s1*q*x and acc0 = sum s0*q*x over the whole
// super-block, and S = 8*acc1 + acc0 exactly.  Smin is an M x 16 by 16 x N
// product per super-block of bsums (|.| <= 2048) and mins (<= 63), done on
// v_mfma_f32_32x32x16_f16: every operand is exact in f16 and every partial
// sum (<= 16 * 2048 * 63 < 2^24) exact in f32, so Smin is exact too.
//
// Tiling.  A workgroup (4 wavefronts) owns a 64 (m) x 128 (n) output tile;
// wavefront w owns columns 32w..32w+31 and both 32-row MFMA tiles, so each
// weight digit operand it builds feeds two MFMAs.  Two workgroups share a CU
// (launch bounds 256, 2), so one's VALU work overlaps the other's MFMAs.
//
// Data movement, per super-block:
//   * the activation rows (Q8_K quants, bsums as f16, d) go global -> LDS by
//     buffer-to-LDS copies (no registers), into a ring of NS stages issued
//     NS - 1 super-blocks ahead; each row's 16-byte quant chunks are
//     XOR-swizzled by the row index, so the fragment reads of 16 consecutive
//     rows hit distinct banks;
//   * each lane loads its own weight column's pieces (the meta piece and the
//     four quant pieces of its half of the super-block) straight into
//     registers, one super-block ahead (two register sets, the loop unrolled
//     by two); in the row-block tile layout the 32 columns of a half-wavefront
//     read four full 128-byte lines per load instruction.
// One explicit wait (this wavefront's copies of the stage and its weight
// registers) and one barrier start each super-block; the copies in flight
// for later stages stay outstanding.
//
// Work items (tile, k-split) are numbered so that all m-tiles and k-splits of
// one n-tile run on the same XCD (workgroups are dealt to the 8 XCDs
// round-robin), where they share that XCD's L2 copy of the weight tile.
//
// Split-K.  When there are too few tiles to fill the CUs, the K loop is cut
// into `splits` ranges of super-blocks.  Each workgroup writes its partial
// tile to the workspace, and a second, small launch (gemm_splitk_reduce)
// sums every tile's partials in split order and writes y -- so the result
// does not depend on which workgroup finished first, and no workgroup waits
// on another.
#include "aq_internal.h"
#include "gemm6_impl.h"

#include <algorithm>

namespace aq {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef unsigned short us2 __attribute__((ext_vector_type(2)));

constexpr int GBN = 128;   // columns (n) per workgroup
constexpr int GBM = 64;    // rows (m) per workgroup: two 32-row MFMA tiles
constexpr int NXCD = 8;
constexpr int TARGET_WG = 256;  // split K until there is a work item per CU
constexpr int NS = 4;           // activation stages in LDS

struct GemmParams {
    const uint8_t *w;  // row-block tiles
    int64_t rb_stride;
    int ng;            // super-blocks per row (= k / 256)
    const int8_t *xq;  // activation planes
    const float *xd;
    const uint16_t *xbs;  // bsums as f16
    float *y;
    int m, n, k;
    int ntm, tiles, splits, kbs, items, per_xcd;
    float *part;   // [tiles][splits][GBM][GBN] partial sums (splits > 1)
    int32_t *S, *Smin;  // integer dump [m][n][ng] or null
};

// LDS of one workgroup: NS stages of quants [64 rows][256] (chunk c of row r
// at chunk c ^ (r & 15)) and bsums [64 rows][16] f16, and NS + 1 slots of d
// [64 rows] (one more than the stages: the epilogue of super-block i, spread
// over step i + 1, reads its d after the copies of stage i + NS started).
struct Lds {
    static constexpr int QS = GBM * 256;
    static constexpr int BS = GBM * 32;
    static constexpr int DS = GBM * 4;
    static constexpr int ND = NS + 1;
    static constexpr int Q0 = 0, B0 = NS * QS, D0 = B0 + NS * BS;
    static constexpr int BYTES = D0 + ND * DS;
};
static_assert(2 * Lds::BYTES <= 160 * 1024, "two workgroups per CU");

// bytes b (each <= 15) times s (<= 7), bytewise without carries: two 16-bit
// lanes per dword (v_pk_mul_lo_u16); m holds s in both 16-bit halves.
__device__ __forceinline__ int pkmul(uint32_t x, uint32_t m) {
    const us2 r = __builtin_bit_cast(us2, x) * __builtin_bit_cast(us2, m);
    return (int)__builtin_bit_cast(uint32_t, r);
}
// byte b of w in both 16-bit halves (v_perm_b32; selector 0x0c gives 0)
__device__ __forceinline__ uint32_t bcast_byte16(uint32_t w, int b) {
    return __builtin_amdgcn_perm(w, w, 0x0c000c00u | (uint32_t)b | ((uint32_t)b << 16));
}
// f16 pair (v, v) for byte b (<= 63) of w: bytes (v, 0x64) are 1024 + v as
// f16, exact, and the packed add of -1024 leaves v exactly.
__device__ __forceinline__ uint32_t f16pair_of_byte(uint32_t w, int b) {
    const uint32_t t = __builtin_amdgcn_perm(0x64646464u, w, 0x04000400u | (uint32_t)b | ((uint32_t)b << 16));
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 r = __builtin_bit_cast(h2, t) + (h2){(_Float16)-1024.0f, (_Float16)-1024.0f};
    return __builtin_bit_cast(uint32_t, r);
}

// The kernel's body for workgroup bid of the launch, on LDS of Lds::BYTES
// (so that another launch can run it beside other work).
template <bool DUMP>
__device__ __forceinline__ void gemm_q4k_body(GemmParams p, uint8_t *lds, int bid) {
    // workgroup -> (tile, split): contiguous ranges per XCD, m-tiles then splits fastest
    const int xcd = bid % NXCD, local = bid / NXCD;
    const int item = xcd * p.per_xcd + local;
    if (local >= p.per_xcd || item >= p.items) return;  // uniform over the workgroup
    const int tile = item / p.splits, split = item - tile * p.splits;
    const int tn = tile / p.ntm, tm = tile - tn * p.ntm;
    const int m0 = tm * GBM;
    const int kb0 = split * p.kbs;
    const int nit = min(p.ng, kb0 + p.kbs) - kb0;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, l32 = lane & 31;
    const int ccol = wave * 32 + l32;  // column within the tile
    const int col = tn * GBN + ccol;
    const bool col_ok = col < p.n;
    const int ng = p.ng, k = p.k;

    // ---- copies and weight loads: raw buffer accesses through wave-uniform
    // descriptors; per-lane offsets are fixed for the whole K loop and the
    // super-block advances the scalar offset only.  Activation rows past m and
    // weight columns past n fall outside the descriptors' ranges and read
    // zeros (their outputs are never stored).
    const rsrc_t rq = buf_rsrc(p.xq, (uint32_t)((int64_t)p.m * k));
    const rsrc_t rbs = buf_rsrc(p.xbs, (uint32_t)((int64_t)p.m * (k / 16) * 2));
    const rsrc_t rdx = buf_rsrc(p.xd, (uint32_t)((int64_t)p.m * ng * 4));
    const int nrb = (p.n + RB - 1) / RB;
    const int rb_here = min(16, nrb - 16 * tn);  // row blocks (8 columns each) of this n-tile
    const rsrc_t rw = buf_rsrc(p.w + (int64_t)16 * tn * p.rb_stride, (uint32_t)(rb_here * p.rb_stride));
    uint32_t qoff[4];  // wave w copies rows 16w..16w+15, four rows per instruction
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = 4 * (4 * wave + i) + (lane >> 4), cp = lane & 15;
        qoff[i] = (uint32_t)((m0 + r) * k + 16 * (cp ^ (r & 15)));
    }
    // waves 0, 1: bsums of rows 32w..32w+31 (32 B a row, two lanes each); waves 2 and 3 both
    // copy the d of the 64 rows (the same bytes to the same place), so every
    // wavefront issues the same number of loads per step
    const uint32_t bsoff = (uint32_t)(((m0 + 32 * (wave & 1) + (lane >> 1)) * (k / 16) + 8 * (lane & 1)) * 2);
    const uint32_t dxoff = (uint32_t)((m0 + lane) * ng * 4);
    // weights: this lane's column is row l32 % 8 of row block 4w + l32 / 8;
    // piece 0 (d, dmin, scales) and quant pieces 1 + 2c + h, c = 0..3
    const uint32_t woff = (uint32_t)((4 * wave + (l32 >> 3)) * p.rb_stride + (l32 & 7) * 16);
    const uint32_t wqoff = woff + 128u * (1 + h);

    // A step issues its loads whether or not super-block kb0 + i exists, so
    // every step waits on the same counts; past the last one the loads go
    // through descriptors of zero bytes (the range check covers the per-lane
    // offset, not the scalar one), so they read zeros without touching
    // memory.  The choice of descriptor is scalar: no per-lane selects.
    const rsrc_t rnone = buf_rsrc(p.xq, 0u);
    auto issue_act = [&](int i) {  // super-block kb0 + i into stage i % NS, its d into slot i % ND
        const int b = kb0 + i;
        const bool live = i < nit;
        uint8_t *q = lds + Lds::Q0 + (i % NS) * Lds::QS;
        const rsrc_t r1 = live ? rq : rnone;
#pragma unroll
        for (int c = 0; c < 4; c++) buf_to_lds16(r1, q + 1024 * (4 * wave + c), qoff[c], b * QK_K);
        if (wave < 2) buf_to_lds16(live ? rbs : rnone, lds + Lds::B0 + (i % NS) * Lds::BS + 1024 * wave, bsoff, b * 32);
        else buf_to_lds4(live ? rdx : rnone, lds + Lds::D0 + (i % Lds::ND) * Lds::DS, dxoff, b * 4);
    };
    auto issue_w = [&](u32x4 &meta, u32x4 (&q)[4], int i) {
        const int soff = (kb0 + i) * 9 * 128;
        const rsrc_t r = i < nit ? rw : rnone;
        meta = __builtin_amdgcn_raw_buffer_load_b128(r, woff, soff, 0);
#pragma unroll
        for (int c = 0; c < 4; c++) q[c] = __builtin_amdgcn_raw_buffer_load_b128(r, wqoff + 256u * c, soff, 0);
    };

    v16f yacc[2];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) yacc[t][r] = 0.0f;

    // Carried from super-block i - 1 into step i: T = d_w * S - dmin_w * Smin
    // per output, formed as soon as the super-block's sums are complete; the
    // remaining  y += d_x * T  is spread over the sub-blocks of step i, one
    // (tile, 4-row group) part after each sub-block's MFMAs.  Before the
    // first super-block T is zero (the parts then add d_x * 0, with d_x read
    // from a filled slot).
    v16f pT[2];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) pT[t][r] = 0.0f;
    const uint8_t *pd = lds + Lds::D0;  // d slot of the carried super-block

    auto epi_part = [&](int q) {  // q = 4 * t + r4: rows 8 * r4 + 4 * h + i of tile t
        const int t = q >> 2, r4 = q & 3;
        const v4f dx4 = *(const v4f *)(pd + 4 * (32 * t + 8 * r4 + 4 * h));
        const float dx[4] = {dx4[0], dx4[1], dx4[2], dx4[3]};
#pragma unroll
        for (int i = 0; i < 4; i++) yacc[t][4 * r4 + i] = __builtin_fmaf(dx[i], pT[t][4 * r4 + i], yacc[t][4 * r4 + i]);
    };

    auto compute = [&](int i, const u32x4 &meta, const u32x4 (&wq)[4]) {
        const uint8_t *qs = lds + Lds::Q0 + (i % NS) * Lds::QS;
        const uint8_t *bsl = lds + Lds::B0 + (i % NS) * Lds::BS;
        // scales / mins of this lane's column (candle's utmp form of get_scale_min_k4)
        const uint32_t u0 = meta.y, u1 = meta.z, u2 = meta.w;
        const uint32_t sc03 = u0 & 0x3F3F3F3Fu;
        const uint32_t sc47 = (u2 & 0x0F0F0F0Fu) | ((u0 >> 2) & 0x30303030u);
        const uint32_t mn03 = u1 & 0x3F3F3F3Fu;
        const uint32_t mn47 = ((u2 >> 4) & 0x0F0F0F0Fu) | ((u1 >> 2) & 0x30303030u);
        const uint32_t dg1[2] = {(sc03 >> 3) & 0x07070707u, (sc47 >> 3) & 0x07070707u};  // s1 per sub-block
        const uint32_t dg0[2] = {sc03 & 0x07070707u, sc47 & 0x07070707u};                // s0 per sub-block
        const float dw = f16_bits_to_f32(meta.x), dmw = f16_bits_to_f32(meta.x >> 16);

        // S = 8 * acc1 + acc0 over the 8 sub-blocks; the A fragments of
        // sub-block j + 1 are read from LDS while the MFMAs of j run.
        auto read_a = [&](v4i (&a)[2], int j) {
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const int R = 32 * t + l32, C = 2 * j + h;
                a[t] = *(const v4i *)(qs + R * 256 + 16 * (C ^ (R & 15)));
            }
        };
        v16i acc1[2], acc0[2];
        v4i abuf[2][2];
        read_a(abuf[0], 0);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const u32x4 pq = wq[j >> 1];
            const uint32_t qv[4] = {pq.x, pq.y, pq.z, pq.w};
            const uint32_t m1 = bcast_byte16(dg1[j >> 2], j & 3), m0s = bcast_byte16(dg0[j >> 2], j & 3);
            v4i d1, d0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t nib = (j & 1) ? (qv[e] >> 4) & 0x0F0F0F0Fu : qv[e] & 0x0F0F0F0Fu;
                d1[e] = pkmul(nib, m1);
                d0[e] = pkmul(nib, m0s);
            }
            if (j < 7) read_a(abuf[(j + 1) & 1], j + 1);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const v16i z = {0};
                acc1[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(abuf[j & 1][t], d1, j == 0 ? z : acc1[t], 0, 0, 0);
                acc0[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(abuf[j & 1][t], d0, j == 0 ? z : acc0[t], 0, 0, 0);
            }
            epi_part(j);  // the previous super-block's part j
        }

        // Smin on f16 MFMA: A[m][g] = bsums (g = 8h + i), B[g][n] = mn[g/2]
        const uint32_t mw = h ? mn47 : mn03;
        const uint32_t bp[4] = {f16pair_of_byte(mw, 0), f16pair_of_byte(mw, 1), f16pair_of_byte(mw, 2),
                                f16pair_of_byte(mw, 3)};
        const v8h bmn = __builtin_bit_cast(v8h, (u32x4){bp[0], bp[1], bp[2], bp[3]});
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const v8h abs = *(const v8h *)(bsl + (32 * t + l32) * 32 + 16 * h);
            const v16f z = {0};
            const v16f sm = __builtin_amdgcn_mfma_f32_32x32x16_f16(abs, bmn, z, 0, 0, 0);
            const v16i S = (acc1[t] << 3) + acc0[t];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                // f32 combine (the tolerance-bound part of the result): fused multiply-add
                pT[t][r] = __builtin_fmaf(-dmw, sm[r], dw * (float)S[r]);
                if (DUMP) {
                    const int row = m0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (row < p.m && col_ok) {
                        const int64_t o = ((int64_t)row * p.n + col) * ng + kb0 + i;
                        p.S[o] = S[r];
                        p.Smin[o] = (int)sm[r];
                    }
                }
            }
        }
        pd = lds + Lds::D0 + (i % Lds::ND) * Lds::DS;
    };

    // The steps.  Before step i: wait for this wavefront's copies of stage i
    // and its weight registers of super-block i (issued before the copies of
    // step i - 1, which may stay in flight), then a barrier, so every
    // wavefront's copies have landed and every wavefront has finished step
    // i - 1, whose stage the copies issued in step i overwrite.
    constexpr int CA = 5;  // loads per copy issue
    auto step = [&](int i, const u32x4 &meta, const u32x4 (&wq)[4], u32x4 &nmeta, u32x4 (&nwq)[4]) {
        issue_w(nmeta, nwq, i + 1);
        issue_act(i + NS - 1);
        compute(i, meta, wq);
        wait_vmcnt<CA>();
        stage_barrier();
    };

    u32x4 meta0, meta1, wq0[4], wq1[4];
    issue_w(meta0, wq0, 0);
#pragma unroll
    for (int i = 0; i < NS - 1; i++) issue_act(i);
    wait_vmcnt<(NS - 2) * CA>();
    stage_barrier();
    for (int i = 0; i < nit; i += 2) {
        step(i, meta0, wq0, meta1, wq1);
        if (i + 1 < nit) step(i + 1, meta1, wq1, meta0, wq0);
    }
#pragma unroll
    for (int q = 0; q < 8; q++) epi_part(q);  // the last super-block's epilogue
    wait_vmcnt<0>();  // the copies issued past the last super-block still write LDS

    if (p.splits == 1) {
        if (col_ok) {
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = m0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (row < p.m) p.y[(int64_t)row * p.n + col] = yacc[t][r];
                }
        }
        return;
    }

    // split-K: publish this partial tile; gemm_splitk_reduce (the next launch
    // on the stream) sums the partials in split order
    float *mine = p.part + ((int64_t)tile * p.splits + split) * (GBM * GBN);
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) mine[(32 * t + 8 * (r >> 2) + 4 * h + (r & 3)) * GBN + ccol] = yacc[t][r];
}

template <bool DUMP>
__global__ __launch_bounds__(256, DUMP ? 1 : 2) void gemm_q4k_kernel(GemmParams p) {
    __shared__ __align__(16) uint8_t lds[Lds::BYTES];
    gemm_q4k_body<DUMP>(p, lds, (int)blockIdx.x);
}

// A Q4_K GEMM and a Q6_K / Q5_K one (T2) on the same activation in one
// launch: workgroups [0, g1) run the first (g1 a multiple of the XCD count,
// so its XCD mapping is kept), the rest the second, on one LDS buffer that
// either body fits.  The first is not split over K; the second may be (its
// partials then go to the workspace and the reduce launch follows).
template <int T2>
__global__ __launch_bounds__(256, 2) void gemm_pair_kernel(GemmParams p1, Gemm6Params p2, int g1) {
    __shared__ __align__(16) uint8_t lds[Lds::BYTES > Lds6::BYTES ? Lds::BYTES : Lds6::BYTES];
    if ((int)blockIdx.x < g1) gemm_q4k_body<false>(p1, lds, (int)blockIdx.x);  // uniform
    else gemm_f16w_body<T2, false>(p2, lds, (int)blockIdx.x - g1);
}

// y = sum over splits (in split order) of the partial tiles; one thread per
// output element of a tile row.  A kernel boundary, not a fence, makes the
// partials visible: a device-scope fence per workgroup costs an L2
// write-back on this GPU.
// V consecutive columns of one tile row per thread (V = 4: 16-byte loads and
// stores, where n % 4 == 0 and y is 16-byte aligned, so that the four stay in
// one output row; the partial tiles are 128 columns wide).  Indices in 32
// bits: the launcher checks that the tiles' elements fit.  The sum starts
// from 0 and adds the parts in order, whatever V.
template <int V>
__global__ __launch_bounds__(256) void gemm_splitk_reduce(const float *__restrict__ part, float *__restrict__ y, int m,
                                                          int n, int ntm, int gbm, int splits, int tiles) {
    const int per_tile = gbm * GBN;
    const int e = ((int)blockIdx.x * 256 + (int)threadIdx.x) * V;
    if (e >= tiles * per_tile) return;
    const int tile = e / per_tile;
    const int w = e - tile * per_tile;
    const int tn = tile / ntm, tm = tile - tn * ntm;
    const int row = tm * gbm + w / GBN, c = tn * GBN + w % GBN;
    if (row >= m || c >= n) return;
    const float *src = part + (int64_t)tile * splits * per_tile + w;
    float *dst = y + (int64_t)row * n + c;
    if (V == 4 && c + 4 <= n) {
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int s2 = 0; s2 < splits; s2++) {
            const float4 t = *(const float4 *)(src + (int64_t)s2 * per_tile);
            acc.x += t.x;
            acc.y += t.y;
            acc.z += t.z;
            acc.w += t.w;
        }
        *(float4 *)dst = acc;
    } else {
        for (int j = 0; j < V && c + j < n; j++) {
            float acc = 0.0f;
            for (int s2 = 0; s2 < splits; s2++) acc += src[(int64_t)s2 * per_tile + j];
            dst[j] = acc;
        }
    }
}

struct GemmPlan {
    int ntm, ntn, tiles, splits, kbs;
    size_t ws;
};

// 64 x 128 tiles, two workgroups per CU; the K loop is split (halves,
// quarters, ...) while there are fewer items than CUs, each split keeping at
// least two super-blocks -- and, from half a CU's worth of items up, at least
// eight: a split of fewer costs more in its reduce launch than the idle CUs
// it fills (512 x 2304 x 2048: 23.4 us in two splits of four super-blocks
// with the reduce, 15.8 us unsplit; 512 x 2048 x 5632: 28.4 us in two
// splits of eleven, 34.9 us unsplit).
GemmPlan gemm_plan(int64_t m, int64_t n, int64_t k) {
    GemmPlan g;
    const int ng = (int)(k / QK_K);
    g.ntn = (int)((n + GBN - 1) / GBN);
    g.ntm = (int)((m + GBM - 1) / GBM);
    g.tiles = g.ntm * g.ntn;
    g.splits = 1;
    while ((int64_t)g.tiles * g.splits < TARGET_WG && ng / (2 * g.splits) >= 2 &&
           ((int64_t)g.tiles * g.splits < TARGET_WG / 2 || ng / (2 * g.splits) >= 8))
        g.splits *= 2;
    g.kbs = (ng + g.splits - 1) / g.splits;
    g.splits = (ng + g.kbs - 1) / g.kbs;
    g.ws = g.splits > 1 ? (size_t)g.tiles * g.splits * GBM * GBN * 4 : 0;
    return g;
}

}  // namespace

// Rows per launch: the copies address the activation planes with 32-bit
// offsets (rows * k < 2^31); longer inputs run as several launches.
static int64_t gemm_chunk_rows(int64_t m, int64_t k) {
    const int64_t cap = (((int64_t)1 << 31) - 1) / k / 128 * 128;
    return m < cap ? m : cap;
}

hipError_t launch_splitk_reduce(const float *part, float *y, int m, int n, int ntm, int gbm, int splits, int tiles,
                                hipStream_t s) {
    const int64_t elems = (int64_t)tiles * gbm * GBN;
    if (elems + 4 * 256 > 0x7fffffff) return hipErrorInvalidValue;
    if (n % 4 == 0 && (((uintptr_t)y | (uintptr_t)part) & 15) == 0)
        gemm_splitk_reduce<4><<<(unsigned)((elems / 4 + 255) / 256), 256, 0, s>>>(part, y, m, n, ntm, gbm, splits, tiles);
    else
        gemm_splitk_reduce<1><<<(unsigned)((elems + 255) / 256), 256, 0, s>>>(part, y, m, n, ntm, gbm, splits, tiles);
    return hipGetLastError();
}

size_t gemm_workspace_bytes(int type, int64_t m, int64_t n, int64_t k) {
    if (type == TYPE_Q6_K || type == TYPE_Q5_K) return gemm6_workspace_bytes(m, n, k);
    if (type == TYPE_Q8_0) return gemm8_workspace_bytes(m, n, k);
    if (type != TYPE_Q4_K || m <= 0 || n <= 0 || k <= 0 || k % QK_K || k > (1 << 24)) return (size_t)-1;
    const int64_t mc = gemm_chunk_rows(m, k);
    const GemmPlan g = gemm_plan(mc, n, k);
    if (g.tiles > GEMM_MAX_TILES) return (size_t)-1;
    size_t ws = g.ws;
    if (m % mc) ws = std::max(ws, gemm_plan(m % mc, n, k).ws);  // the last, shorter launch
    return ws;
}

hipError_t launch_gemm(const WLayout &w, int64_t n, int64_t k, const ActPlanes &x, int64_t m, float *y, int32_t *S,
                       int32_t *Smin, void *ws, size_t ws_bytes, hipStream_t s) {
    if (w.type == TYPE_Q6_K || w.type == TYPE_Q5_K) return launch_gemm6(w, n, k, x, m, y, S, Smin, ws, ws_bytes, s);
    if (w.type == TYPE_Q8_0) return launch_gemm8(w, n, k, x, m, y, S, Smin, ws, ws_bytes, s);
    if (w.type != TYPE_Q4_K) return hipErrorNotSupported;
    if (!w.slab || !y || !x.qs || !x.d || !x.bsum16 || m <= 0 || n <= 0 || k <= 0 || k % QK_K) return hipErrorInvalidValue;
    if (m > 0x7fffffff || n > 0x7fffffff || k > (1 << 24) || w.ng != k / QK_K) return hipErrorInvalidValue;
    if ((int64_t)16 * w.rb_stride >= ((int64_t)1 << 31)) return hipErrorNotSupported;  // one n-tile's weights
    if ((S == nullptr) != (Smin == nullptr)) return hipErrorInvalidValue;
    const int64_t mc = gemm_chunk_rows(m, k);
    const int ng = w.ng;
    for (int64_t r0 = 0; r0 < m; r0 += mc) {
        const int64_t mm = std::min(mc, m - r0);
        const GemmPlan g = gemm_plan(mm, n, k);
        if (g.tiles > GEMM_MAX_TILES) return hipErrorNotSupported;
        if (g.splits > 1 && (!ws || ws_bytes < g.ws)) return hipErrorInvalidValue;
        GemmParams p;
        p.w = w.slab;
        p.rb_stride = w.rb_stride;
        p.ng = ng;
        p.xq = x.qs + r0 * k;
        p.xd = x.d + r0 * ng;
        p.xbs = x.bsum16 + r0 * (k / 16);
        p.y = y + r0 * n;
        p.m = (int)mm;
        p.n = (int)n;
        p.k = (int)k;
        p.ntm = g.ntm;
        p.tiles = g.tiles;
        p.splits = g.splits;
        p.kbs = g.kbs;
        p.items = g.tiles * g.splits;
        p.per_xcd = (p.items + NXCD - 1) / NXCD;
        p.part = (float *)ws;
        p.S = S ? S + r0 * n * ng : nullptr;
        p.Smin = Smin ? Smin + r0 * n * ng : nullptr;
        const unsigned grid = (unsigned)(p.per_xcd * NXCD);
        if (S) gemm_q4k_kernel<true><<<grid, 256, 0, s>>>(p);
        else gemm_q4k_kernel<false><<<grid, 256, 0, s>>>(p);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (g.splits > 1 && (e = launch_splitk_reduce(p.part, p.y, p.m, p.n, g.ntm, GBM, g.splits, g.tiles, s)) != hipSuccess)
            return e;
    }
    return hipSuccess;
}

hipError_t launch_gemm_pair(const WLayout &w1, int64_t n1, float *y1, const WLayout &w2, int64_t n2, float *y2,
                            int64_t k, const ActPlanes &x, int64_t m, void *ws, size_t ws_bytes, hipStream_t s) {
    if (w1.type != TYPE_Q4_K || (w2.type != TYPE_Q6_K && w2.type != TYPE_Q5_K)) return hipErrorNotSupported;
    const bool q5 = w2.type == TYPE_Q5_K;
    if (!w1.slab || !w2.slab || (!q5 && !w2.d) || !y1 || !y2 || !x.qs || !x.d || !x.bsum16) return hipErrorInvalidValue;
    if (!x.q16) return hipErrorNotSupported;  // the second GEMM reads the f16 quants the quantizer wrote
    if (m <= 0 || n1 <= 0 || n2 <= 0 || k <= 0 || k % QK_K || m > 0x7fffffff || n1 > 0x7fffffff ||
        n2 > 0x7fffffff || k > (1 << 24) || w1.ng != k / QK_K || w2.ng != k / QK_K)
        return hipErrorInvalidValue;
    if ((int64_t)16 * w1.rb_stride >= ((int64_t)1 << 31) || (int64_t)16 * w2.rb_stride >= ((int64_t)1 << 31))
        return hipErrorNotSupported;
    // one launch of each (no row chunks), the first unsplit, the second split
    // as its own launch would be, and together no more workgroups than the
    // CUs hold at once
    if (gemm_chunk_rows(m, k) < m || gemm6_chunk_rows(k) < m) return hipErrorNotSupported;
    GemmPlan g1 = gemm_plan(m, n1, k);
    Gemm6Plan g2 = gemm6_plan(m, n2, k);
    if ((int64_t)g1.tiles + (int64_t)g2.tiles * g2.splits > TARGET_WG6 || g1.tiles > GEMM_MAX_TILES ||
        g2.tiles > GEMM_MAX_TILES)
        return hipErrorNotSupported;
    if (g2.splits > 1 && (!ws || ws_bytes < g2.part)) return hipErrorInvalidValue;
    const int ng = w1.ng;
    GemmParams p;
    p.w = w1.slab;
    p.rb_stride = w1.rb_stride;
    p.ng = ng;
    p.xq = x.qs;
    p.xd = x.d;
    p.xbs = x.bsum16;
    p.y = y1;
    p.m = (int)m;
    p.n = (int)n1;
    p.k = (int)k;
    p.ntm = g1.ntm;
    p.tiles = g1.tiles;
    p.splits = 1;
    p.kbs = ng;
    p.items = g1.tiles;
    p.per_xcd = (p.items + NXCD - 1) / NXCD;
    p.part = nullptr;
    p.S = p.Smin = nullptr;
    Gemm6Params q;
    q.w = w2.slab;
    q.wd = w2.d;
    q.rb_stride = w2.rb_stride;
    q.ng = ng;
    q.x16 = x.q16;
    q.xd = x.d;
    q.xbs = q5 ? x.bsum16 : nullptr;
    q.y = y2;
    q.m = (int)m;
    q.n = (int)n2;
    q.k = (int)k;
    q.ntm = g2.ntm;
    q.tiles = g2.tiles;
    q.splits = g2.splits;
    q.kbs = g2.kbs;
    q.items = g2.tiles * g2.splits;
    q.per_xcd = (q.items + NXCD6 - 1) / NXCD6;
    q.part = (float *)ws;
    q.S = q.Smin = nullptr;
    const int b1 = p.per_xcd * NXCD, b2 = q.per_xcd * NXCD6;
    if (q5) gemm_pair_kernel<TYPE_Q5_K><<<(unsigned)(b1 + b2), 256, 0, s>>>(p, q, b1);
    else gemm_pair_kernel<TYPE_Q6_K><<<(unsigned)(b1 + b2), 256, 0, s>>>(p, q, b1);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || g2.splits == 1) return e;
    return launch_splitk_reduce(q.part, y2, q.m, q.n, g2.ntm, G6M, g2.splits, g2.tiles, s);
}

}  // namespace aq
