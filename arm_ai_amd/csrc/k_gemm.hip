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
// Tiling.  A workgroup (4 wavefronts) owns a 32*MT (m) x 128 (n) output
// tile; wavefront w owns columns 32w..32w+31 and all rows (MT 32x32 MFMA
// tiles), so each weight digit operand it builds is used MT times.  The
// activation rows of two super-blocks at a time (quants, bsums, d) are copied
// global -> LDS directly (global_load_lds, no registers), double-buffered, the
// 16-byte quant chunks of each row XOR-swizzled so that 16 consecutive rows
// read distinct banks.  Each lane loads its own weight column's pieces (the
// meta piece and the four quant pieces of its half of the super-block) into
// registers one stage ahead; in the row-block tile layout the 32 columns of a
// wavefront's half read 4 full 128-byte lines per instruction.
// Work items (tile, k-split) are numbered so that all m-tiles and k-splits of
// one n-tile run on the same XCD (workgroups are dealt to the 8 XCDs
// round-robin), where they share that XCD's L2 copy of the weight tile.
//
// Split-K.  When there are too few tiles to fill the 256 CUs, the K loop is
// cut into `splits` ranges of super-blocks.  Each workgroup writes its partial
// tile to the workspace, and a second, small launch (gemm_splitk_reduce)
// sums every tile's partials in split order and writes y -- so the result
// does not depend on which workgroup finished first, and no workgroup waits
// on another.
#include "aq_internal.h"

#include <algorithm>

namespace aq {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef unsigned short us2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int GBN = 128;   // columns (n) per workgroup
constexpr int NXCD = 8;
constexpr int TARGET_WG = 256;  // split K until there is a work item per CU

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
    float *part;   // [tiles][splits][32*MT][GBN] partial sums (splits > 1)
    int32_t *S, *Smin;  // integer dump [m][n][ng] or null
};

// bytes b (each <= 15) times s (<= 7), bytewise without carries: two 16-bit
// lanes per dword (v_pk_mul_lo_u16).
__device__ __forceinline__ int pkmul(uint32_t x, uint32_t s) {
    const us2 a = __builtin_bit_cast(us2, x);
    const us2 r = a * (us2){(unsigned short)s, (unsigned short)s};
    return (int)__builtin_bit_cast(uint32_t, r);
}

// LDS of one workgroup (a tile of 32*MT rows x GBN columns):
//   two main stages, one super-block each:
//     quants [rows][256] i8, 16-byte chunk c of row r at chunk c ^ (r & 15), so
//       the 16-byte reads of 16 consecutive rows hit distinct banks;
//     weight pieces [9][GBN columns][16 B] (piece 0: d, dmin, scales; 1..8:
//       qs), each piece padded by 64 B so the half-wavefronts' reads of pieces
//       1 + 2c and 2 + 2c start on different banks;
//   three small stages (a ring), one super-block each:
//     bsums [rows][16] as f16;
//     d: one 256-byte slot per 32 rows, row 32s + i at slot s entry i (entries
//       32..63 receive duplicates).
// The ring is one stage deeper than the main stages because the f32 epilogue
// of super-block b runs during step b + 1, after the copies for b + 2 started.
template <int MT>
struct TileLds {
    static constexpr int ROWS = 32 * MT;
    static constexpr int QS = ROWS * 256;
    static constexpr int BP = GBN * 16 + 64;
    static constexpr int MAIN = QS + 9 * BP;  // one main stage; weights at QS
    static constexpr int BS = ROWS * 32, DS = MT * 256;
    static constexpr int SMALL = BS + DS;     // one ring stage; d at BS
    static constexpr int RING0 = 2 * MAIN;
    static constexpr int BYTES = RING0 + 3 * SMALL;
};

template <int MT, bool DUMP>
__global__ __launch_bounds__(256, 2) void gemm_q4k_kernel(GemmParams p) {
    static_assert(MT == 2, "the epilogue is spread as one (tile, 4-row group) part per sub-block");
    constexpr int GBM = 32 * MT;
    using TL = TileLds<MT>;
    __shared__ __align__(16) uint8_t lds[TL::BYTES];

    // workgroup -> (tile, split): contiguous ranges per XCD, m-tiles then splits fastest
    const int xcd = blockIdx.x % NXCD, local = blockIdx.x / NXCD;
    const int item = xcd * p.per_xcd + local;
    if (local >= p.per_xcd || item >= p.items) return;  // uniform over the workgroup
    const int tile = item / p.splits, split = item - tile * p.splits;
    const int tn = tile / p.ntm, tm = tile - tn * p.ntm;
    const int m0 = tm * GBM;
    const int kb0 = split * p.kbs;
    const int kb1 = min(p.ng, kb0 + p.kbs);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, l32 = lane & 31;
    const int ccol = wave * 32 + l32;  // column within the tile
    const int col = tn * GBN + ccol;
    const bool col_ok = col < p.n;
    const int ng = p.ng, k = p.k;

    // ---- the copies: raw buffer loads into LDS through wave-uniform
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
    uint32_t qoff[2 * MT];
#pragma unroll
    for (int i = 0; i < 2 * MT; i++) {
        const int r = 4 * (2 * MT * wave + i) + (lane >> 4), cp = lane & 15;
        qoff[i] = (uint32_t)((m0 + r) * k + 16 * (cp ^ (r & 15)));
    }
    const int s32 = wave % MT;  // 32-row slice this wave copies bsums and d for (waves < MT)
    const uint32_t bsoff = (uint32_t)(((m0 + 32 * s32 + (lane >> 1)) * (k / 16) + 8 * (lane & 1)) * 2);
    const uint32_t dxoff = (uint32_t)((m0 + 32 * s32 + (lane & 31)) * ng * 4);
    // weight copy (piece, half): lane L loads the 16 bytes of column 64*half + L,
    // i.e. row (L % 8) of this n-tile's row block 8*half + L/8
    const uint32_t woff0 = (uint32_t)((lane >> 3) * p.rb_stride + (lane & 7) * 16);
    const uint32_t woff1 = woff0 + (uint32_t)(8 * p.rb_stride);

    auto issue = [&](uint8_t *main, uint8_t *ring, int b) {
#pragma unroll
        for (int i = 0; i < 2 * MT; i++) buf_to_lds16(rq, main + 1024 * (2 * MT * wave + i), qoff[i], b * QK_K);
        if (wave < MT) {  // wave-uniform
            buf_to_lds16(rbs, ring + 1024 * s32, bsoff, b * 32);
            buf_to_lds4(rdx, ring + TL::BS + 256 * s32, dxoff, b * 4);
        }
        for (int c = wave; c < 18; c += 4) {  // wave-uniform
            const int piece = c >> 1, half = c & 1;
            buf_to_lds16(rw, main + TL::QS + piece * TL::BP + 1024 * half, half ? woff1 : woff0, (b * 9 + piece) * 128);
        }
    };

    v16f yacc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) yacc[t][r] = 0.0f;

    // Carried from super-block b - 1 into step b: its exact integer sums and
    // scales; its f32 epilogue  y += d_x * (d_w * S - dmin_w * Smin)  is spread
    // over the sub-blocks of b, one (tile, 4-row group) part after each
    // sub-block's MFMAs, so the VALU work overlaps the matrix cores.  Before
    // the first super-block the carried sums and scales are zero (the parts
    // then add d_x * 0, with d_x read from a stage that holds real data).
    v16i pS[MT];
    v16f pSm[MT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            pS[t][r] = 0;
            pSm[t][r] = 0.0f;
        }
    float pdw = 0.0f, pdmw = 0.0f;
    const uint8_t *pring = lds + TL::RING0;
    int pb = -1;

    auto epi_part = [&](int q) {  // q = 4 * t + r4: rows 8 * r4 + 4 * h + i of tile t
        const int t = q >> 2, r4 = q & 3;
        const v4f dx4 = *(const v4f *)(pring + TL::BS + 256 * t + 4 * (8 * r4 + 4 * h));
        const float dx[4] = {dx4[0], dx4[1], dx4[2], dx4[3]};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 4 * r4 + i;
            // f32 combine (the tolerance-bound part of the result): fused multiply-adds
            yacc[t][r] = __builtin_fmaf(dx[i], __builtin_fmaf(-pdmw, pSm[t][r], pdw * (float)pS[t][r]), yacc[t][r]);
            if (DUMP) {
                const int row = m0 + 32 * t + 8 * r4 + 4 * h + i;
                if (pb >= 0 && row < p.m && col_ok) {
                    const int64_t o = ((int64_t)row * p.n + col) * ng + pb;
                    p.S[o] = pS[t][r];
                    p.Smin[o] = (int)pSm[t][r];
                }
            }
        }
    };

    auto compute = [&](const uint8_t *main, const uint8_t *ring, int b) {
        // this lane's column: piece 0 and the four quant pieces of its half
        const uint8_t *wp = main + TL::QS + ccol * 16;
        const u32x4 meta = *(const u32x4 *)wp;
        u32x4 bq[4];
#pragma unroll
        for (int c = 0; c < 4; c++) bq[c] = *(const u32x4 *)(wp + (1 + 2 * c + h) * TL::BP);
        // scales / mins of this lane's column (candle's utmp form of get_scale_min_k4)
        const uint32_t u0 = meta.y, u1 = meta.z, u2 = meta.w;
        const uint32_t sc03 = u0 & 0x3F3F3F3Fu;
        const uint32_t sc47 = (u2 & 0x0F0F0F0Fu) | (((u0 >> 6) & 0x03030303u) << 4);
        const uint32_t mn03 = u1 & 0x3F3F3F3Fu;
        const uint32_t mn47 = ((u2 >> 4) & 0x0F0F0F0Fu) | (((u1 >> 6) & 0x03030303u) << 4);
        const float dw = f16_bits_to_f32(meta.x), dmw = f16_bits_to_f32(meta.x >> 16);

        // S = 8 * acc1 + acc0 over the 8 sub-blocks; the A fragments of
        // sub-block j + 1 are read from LDS while the MFMAs of j run.
        auto read_a = [&](v4i (&a)[MT], int j) {
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const int R = 32 * t + l32, C = 2 * j + h;
                a[t] = *(const v4i *)(main + R * 256 + 16 * (C ^ (R & 15)));
            }
        };
        v16i acc1[MT], acc0[MT];
        v4i abuf[2][MT];
        read_a(abuf[0], 0);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const u32x4 pq = bq[j >> 1];
            const uint32_t qv[4] = {pq.x, pq.y, pq.z, pq.w};
            const uint32_t sw = j < 4 ? sc03 : sc47;
            const uint32_t sc = (sw >> (8 * (j & 3))) & 0xffu;
            const uint32_t s1 = sc >> 3, s0 = sc & 7u;
            v4i d1, d0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t nib = (j & 1) ? (qv[i] >> 4) & 0x0F0F0F0Fu : qv[i] & 0x0F0F0F0Fu;
                d1[i] = pkmul(nib, s1);
                d0[i] = pkmul(nib, s0);
            }
            if (j < 7) read_a(abuf[(j + 1) & 1], j + 1);
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const v16i z = {0};
                acc1[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(abuf[j & 1][t], d1, j == 0 ? z : acc1[t], 0, 0, 0);
                acc0[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(abuf[j & 1][t], d0, j == 0 ? z : acc0[t], 0, 0, 0);
            }
            epi_part(j);  // the previous super-block's part j
        }

        // Smin of b on f16 MFMA: A[m][g] = bsums (g = 8h + i), B[g][n] = mn[g/2]
        const uint32_t mw = h ? mn47 : mn03;
        v8h bmn;
#pragma unroll
        for (int i = 0; i < 8; i++) bmn[i] = (_Float16)(int)((mw >> (8 * (i >> 1))) & 0xffu);
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const v8h abs = *(const v8h *)(ring + (32 * t + l32) * 32 + 16 * h);
            const v16f z = {0};
            pSm[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(abs, bmn, z, 0, 0, 0);
            pS[t] = (acc1[t] << 3) + acc0[t];
        }
        pdw = dw;
        pdmw = dmw;
        pring = ring;
        pb = b;
    };

    // Main stages alternate, ring stages rotate over three.  The copies for
    // super-block b + 1 are issued right after the barrier and have the
    // compute of b to land; each step begins by waiting for this wave's
    // outstanding copies (only those of the stage about to be read are
    // outstanding by then).  At step b the copies overwrite the main stage
    // of b - 1 (read during step b - 1) and the ring stage of b - 2 (whose
    // epilogue ran during step b - 1).
    issue(lds, lds + TL::RING0, kb0);
    for (int b = kb0; b < kb1; b++) {
        const int i = b - kb0;
        uint8_t *main = lds + (i & 1) * TL::MAIN;
        uint8_t *ring = lds + TL::RING0 + (i % 3) * TL::SMALL;
        if (i == 0) pring = ring;  // the first parts read real d_x and add d_x * 0
        wait_vmcnt<0>();
        stage_barrier();
        if (b + 1 < kb1)
            issue(lds + ((i + 1) & 1) * TL::MAIN, lds + TL::RING0 + ((i + 1) % 3) * TL::SMALL, b + 1);
        compute(main, ring, b);
    }
#pragma unroll
    for (int q = 0; q < 4 * MT; q++) epi_part(q);  // the last super-block's epilogue
    stage_barrier();  // the split-K tail below reuses no stage, but keeps waves together

    if (p.splits == 1) {
        if (col_ok) {
#pragma unroll
            for (int t = 0; t < MT; t++)
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
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) mine[(32 * t + 8 * (r >> 2) + 4 * h + (r & 3)) * GBN + ccol] = yacc[t][r];
}

// y = sum over splits (in split order) of the partial tiles; one thread per
// output element of a tile row.  A kernel boundary, not a fence, makes the
// partials visible: a device-scope fence per workgroup costs an L2
// write-back on this GPU.
__global__ __launch_bounds__(256) void gemm_splitk_reduce(const float *__restrict__ part, float *__restrict__ y, int m,
                                                          int n, int ntm, int gbm, int splits, int tiles) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per_tile = (int64_t)gbm * GBN;
    if (e >= (int64_t)tiles * per_tile) return;
    const int tile = (int)(e / per_tile);
    const int w = (int)(e - (int64_t)tile * per_tile);
    const int tn = tile / ntm, tm = tile - tn * ntm;
    const int row = tm * gbm + w / GBN, c = tn * GBN + w % GBN;
    if (row >= m || c >= n) return;
    const float *src = part + (int64_t)tile * splits * per_tile + w;
    float acc = 0.0f;
    for (int s2 = 0; s2 < splits; s2++) acc += src[(int64_t)s2 * per_tile];
    y[(int64_t)row * n + c] = acc;
}

struct GemmPlan {
    int ntm, ntn, tiles, splits, kbs;
    size_t ws;
};

// 64 x 128 tiles, two workgroups per CU (their wavefronts share the SIMDs but
// not their barriers, so one's VALU epilogue overlaps the other's MFMAs);
// the K loop is split (halves, quarters, ...) while there are fewer items than
// CUs, each split keeping at least two super-blocks.
GemmPlan gemm_plan(int64_t m, int64_t n, int64_t k) {
    GemmPlan g;
    const int ng = (int)(k / QK_K);
    const int gbm = 32 * 2;
    g.ntn = (int)((n + GBN - 1) / GBN);
    g.ntm = (int)((m + gbm - 1) / gbm);
    g.tiles = g.ntm * g.ntn;
    g.splits = 1;
    while ((int64_t)g.tiles * g.splits < TARGET_WG && ng / (2 * g.splits) >= 2) g.splits *= 2;
    g.kbs = (ng + g.splits - 1) / g.splits;
    g.splits = (ng + g.kbs - 1) / g.kbs;
    g.ws = g.splits > 1 ? (size_t)g.tiles * g.splits * gbm * GBN * 4 : 0;
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
    gemm_splitk_reduce<<<(unsigned)((elems + 255) / 256), 256, 0, s>>>(part, y, m, n, ntm, gbm, splits, tiles);
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

uint16_t *gemm_q16_plane(int type, int64_t m, int64_t n, int64_t k, void *ws) {
    return type == TYPE_Q6_K || type == TYPE_Q5_K ? gemm6_q16_plane(m, n, k, ws) : nullptr;
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
        if (S) gemm_q4k_kernel<2, true><<<grid, 256, 0, s>>>(p);
        else gemm_q4k_kernel<2, false><<<grid, 256, 0, s>>>(p);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (g.splits > 1) {
            const int64_t elems = (int64_t)g.tiles * 64 * GBN;
            gemm_splitk_reduce<<<(unsigned)((elems + 255) / 256), 256, 0, s>>>(p.part, p.y, p.m, p.n, g.ntm, 64, g.splits,
                                                                             g.tiles);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

}  // namespace aq
