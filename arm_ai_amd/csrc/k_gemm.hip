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
// tile to the workspace and bumps the tile's counter; the workgroup that
// arrives last (no one waits) sums the partials in split order -- so the
// result does not depend on arrival order -- writes y, and resets the counter
// to zero for the next launch.
#include "aq_internal.h"

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
constexpr int TARGET_WG = 256;  // at least one workgroup per CU

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
    int *counters; // [tiles], zero between launches
    int32_t *S, *Smin;  // integer dump [m][n][ng] or null
};

// bytes b (each <= 15) times s (<= 7), bytewise without carries: two 16-bit
// lanes per dword (v_pk_mul_lo_u16).
__device__ __forceinline__ int pkmul(uint32_t x, uint32_t s) {
    const us2 a = __builtin_bit_cast(us2, x);
    const us2 r = a * (us2){(unsigned short)s, (unsigned short)s};
    return (int)__builtin_bit_cast(uint32_t, r);
}

struct BStage {
    uint4 meta;
    uint4 q[4];  // piece 1 + 2c + h, c = 0..3 (h = this lane's half)
};

typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(1))) void glob_void;

// One activation stage in LDS: 32*MT rows of SB = 2 consecutive super-blocks.
// Per super-block (SUB bytes apart):
//   quants [rows][256]: 16-byte chunk c of row r stored at chunk c ^ (r & 15),
//     so the 16-byte reads of 16 consecutive rows hit distinct banks;
//   bsums [rows][16] i16;
//   d: one 256-byte slot per 32 rows, row 32s + i at slot s entry i (entries
//     32..63 receive duplicates).
template <int MT>
struct AStageLds {
    static constexpr int SB = 2;
    static constexpr int ROWS = 32 * MT;
    static constexpr int QS = ROWS * 256, BS = ROWS * 32, DS = MT * 256;
    static constexpr int SUB = QS + BS + DS;
    static constexpr int BYTES = SB * SUB;
};

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0], expcnt[6:4],
// lgkmcnt[11:8], vmcnt[5:4] at [15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier without the memory fence __syncthreads() adds (that
// fence would wait for every outstanding copy, including the ones issued
// ahead for later stages).  The "memory" clobber keeps the compiler from
// moving loads and stores across it; completion of the copies a stage needs
// is waited for explicitly with wait_vmcnt before it.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <int MT, bool DUMP>
__global__ __launch_bounds__(256, MT == 4 ? 1 : 2) void gemm_q4k_kernel(GemmParams p) {
    constexpr int GBM = 32 * MT;
    using ST = AStageLds<MT>;
    __shared__ __align__(16) uint8_t L0[ST::BYTES];
    __shared__ __align__(16) uint8_t L1[ST::BYTES];
    __shared__ int last_flag;

    // workgroup -> (tile, split): contiguous ranges per XCD, m-tiles then splits fastest
    const int xcd = blockIdx.x % NXCD, local = blockIdx.x / NXCD;
    const int item = xcd * p.per_xcd + local;
    if (local >= p.per_xcd || item >= p.items) return;  // uniform over the workgroup
    const int tile = item / p.splits, split = item - tile * p.splits;
    const int tn = tile / p.ntm, tm = tile - tn * p.ntm;
    const int m0 = tm * GBM;
    const int kb0 = split * p.kbs;
    const int kb1 = min(p.ng, kb0 + p.kbs);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, l32 = lane & 31;
    const int ccol = wave * 32 + l32;  // column within the tile
    const int col = tn * GBN + ccol;
    const bool col_ok = col < p.n;
    const int ng = p.ng, k = p.k;

    // ---- activation stage: direct global -> LDS copies, no registers.
    // Rows past m copy row m-1 (their outputs are never stored).
    // Per-lane source rows of the copies (rows past m copy row m-1, whose
    // outputs are never stored), computed once.
    const int8_t *qsrc[2 * MT];
#pragma unroll
    for (int i = 0; i < 2 * MT; i++) {
        const int r = 4 * (2 * MT * wave + i) + (lane >> 4), cp = lane & 15;
        qsrc[i] = p.xq + (int64_t)min(m0 + r, p.m - 1) * k + 16 * (cp ^ (r & 15));
    }
    const int s32 = wave % MT;  // 32-row slice this wave copies bsums and d for
    const uint16_t *bsrc = p.xbs + (int64_t)min(m0 + 32 * s32 + (lane >> 1), p.m - 1) * (k / 16) + 8 * (lane & 1);
    const float *dsrc = p.xd + (int64_t)min(m0 + 32 * s32 + (lane & 31), p.m - 1) * ng;
    // ---- activation stage: direct global -> LDS copies, no registers.
    auto dma_a = [&](uint8_t *stage, int b) {
#pragma unroll
        for (int i = 0; i < 2 * MT; i++)
            __builtin_amdgcn_global_load_lds((glob_void *)(qsrc[i] + b * QK_K),
                                             (lds_void *)(stage + 1024 * (2 * MT * wave + i)), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((glob_void *)(bsrc + b * 16), (lds_void *)(stage + ST::QS + 1024 * s32), 16,
                                         0, 0);
        __builtin_amdgcn_global_load_lds((glob_void *)(dsrc + b), (lds_void *)(stage + ST::QS + ST::BS + 256 * s32), 4,
                                         0, 0);
    };
    // ---- weight pieces of this lane's column (plain loads: the m-tiles of an
    // n-tile reuse them from L2).  Columns past n load column 0 (never stored).
    const int wc = col_ok ? col : 0;
    const uint8_t *wcol = p.w + (int64_t)(wc >> 3) * p.rb_stride + (wc & 7) * 16;  // + (9 b + piece) * 128
    auto load_b = [&](BStage &st, int b) {
        const uint8_t *wb = wcol + (int64_t)b * (9 * 128);
        st.meta = *(const uint4 *)wb;
#pragma unroll
        for (int c = 0; c < 4; c++) st.q[c] = *(const uint4 *)(wb + (1 + 2 * c + h) * 128);
    };

    v16f yacc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) yacc[t][r] = 0.0f;

    auto compute = [&](const uint8_t *stage, const BStage &bc, int b) {
        // scales / mins of this lane's column (candle's utmp form of get_scale_min_k4)
        const uint32_t u0 = bc.meta.y, u1 = bc.meta.z, u2 = bc.meta.w;
        const uint32_t sc03 = u0 & 0x3F3F3F3Fu;
        const uint32_t sc47 = (u2 & 0x0F0F0F0Fu) | (((u0 >> 6) & 0x03030303u) << 4);
        const uint32_t mn03 = u1 & 0x3F3F3F3Fu;
        const uint32_t mn47 = ((u2 >> 4) & 0x0F0F0F0Fu) | (((u1 >> 6) & 0x03030303u) << 4);
        const float dw = f16_bits_to_f32(bc.meta.x), dmw = f16_bits_to_f32(bc.meta.x >> 16);

        // S = 8 * acc1 + acc0 over the 8 sub-blocks; the A fragments of
        // sub-block j + 1 are read from LDS while the MFMAs of j run.
        auto read_a = [&](v4i (&a)[MT], int j) {
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const int R = 32 * t + l32, C = 2 * j + h;
                a[t] = *(const v4i *)(stage + R * 256 + 16 * (C ^ (R & 15)));
            }
        };
        v16i acc1[MT], acc0[MT];
        v4i abuf[2][MT];
        read_a(abuf[0], 0);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint4 pq = bc.q[j >> 1];
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
        }

        // Smin on f16 MFMA: A[m][g] = bsums (g = 8h + i), B[g][n] = mn[g/2]
        const uint32_t mw = h ? mn47 : mn03;
        v8h bmn;
#pragma unroll
        for (int i = 0; i < 8; i++) bmn[i] = (_Float16)(int)((mw >> (8 * (i >> 1))) & 0xffu);
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const v8h abs = *(const v8h *)(stage + ST::QS + (32 * t + l32) * 32 + 16 * h);
            const v16f z = {0};
            const v16f smin = __builtin_amdgcn_mfma_f32_32x32x16_f16(abs, bmn, z, 0, 0, 0);

            // epilogue of this super-block: y += d_x * (d_w * S - dmin_w * Smin)
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++) {
                const v4f dx4 = *(const v4f *)(stage + ST::QS + ST::BS + 256 * t + 4 * (8 * r4 + 4 * h));
                const float dx[4] = {dx4[0], dx4[1], dx4[2], dx4[3]};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 4 * r4 + i;
                    const int S = (acc1[t][r] << 3) + acc0[t][r];
                    // f32 combine (the tolerance-bound part of the result): fused multiply-adds
                    yacc[t][r] = __builtin_fmaf(dx[i], __builtin_fmaf(-dmw, smin[r], dw * (float)S), yacc[t][r]);
                    if (DUMP) {
                        const int row = m0 + 32 * t + 8 * r4 + 4 * h + i;
                        if (row < p.m && col_ok) {
                            const int64_t o = ((int64_t)row * p.n + col) * ng + b;
                            p.S[o] = S;
                            p.Smin[o] = (int)smin[r];
                        }
                    }
                }
            }
        }
    };

    // Two stages of two super-blocks each.  The copies for the next stage
    // are issued right after the barrier and have the whole compute of the
    // current stage (two super-blocks) to land; each step begins by waiting
    // for all of this wave's outstanding copies, so the wait never stalls on
    // copies issued for a later stage.
    BStage Bc[2], Bn[2];
    auto issue = [&](uint8_t *stage, BStage (&bs)[2], int b) {
#pragma unroll
        for (int u = 0; u < ST::SB; u++) {
            if (b + u < kb1) {
                dma_a(stage + u * ST::SUB, b + u);
                load_b(bs[u], b + u);
            }
        }
    };
    auto step = [&](const uint8_t *cur, const BStage (&bcur)[2], uint8_t *nxt, BStage (&bnxt)[2], int b) {
        wait_vmcnt<0>();
        stage_barrier();  // every wave's copies into `cur` landed; `nxt` (the stage before) is free
        if (b + ST::SB < kb1) issue(nxt, bnxt, b + ST::SB);
#pragma unroll
        for (int u = 0; u < ST::SB; u++)
            if (b + u < kb1) compute(cur + u * ST::SUB, bcur[u], b + u);
    };
    issue(L0, Bc, kb0);
    for (int b = kb0; b < kb1; b += 2 * ST::SB) {
        step(L0, Bc, L1, Bn, b);
        if (b + ST::SB < kb1) step(L1, Bn, L0, Bc, b + ST::SB);
    }
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

    // split-K: publish this partial tile, the last arriving workgroup reduces
    float *mine = p.part + ((int64_t)tile * p.splits + split) * (GBM * GBN);
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) mine[(32 * t + 8 * (r >> 2) + 4 * h + (r & 3)) * GBN + ccol] = yacc[t][r];
    __threadfence();
    __syncthreads();
    if (tid == 0) last_flag = atomicAdd(&p.counters[tile], 1) == p.splits - 1;
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
    const float *all = p.part + (int64_t)tile * p.splits * (GBM * GBN);
    for (int e = tid; e < GBM * GBN; e += 256) {
        const int row = m0 + e / GBN, c = tn * GBN + e % GBN;
        float acc = 0.0f;
        for (int s2 = 0; s2 < p.splits; s2++) acc += all[(int64_t)s2 * (GBM * GBN) + e];
        if (row < p.m && c < p.n) p.y[(int64_t)row * p.n + c] = acc;
    }
    if (tid == 0) p.counters[tile] = 0;
}

struct GemmPlan {
    int mt, ntm, ntn, tiles, splits, kbs;
    size_t ws;
};

GemmPlan gemm_plan(int64_t m, int64_t n, int64_t k) {
    GemmPlan g;
    const int ng = (int)(k / QK_K);
    g.ntn = (int)((n + GBN - 1) / GBN);
    // 128-row tiles reuse each weight digit operand 4 times; take them when
    // they still give every CU a workgroup, else 64-row tiles.
    g.mt = (int64_t)((m + 127) / 128) * g.ntn >= TARGET_WG ? 4 : 2;
    g.ntm = (int)((m + 32 * g.mt - 1) / (32 * g.mt));
    g.tiles = g.ntm * g.ntn;
    // split the K loop only when even 64-row tiles leave most CUs idle
    g.splits = 1;
    while ((int64_t)g.tiles * g.splits < TARGET_WG / 2 && ng / (2 * g.splits) >= 2) g.splits *= 2;
    g.kbs = (ng + g.splits - 1) / g.splits;
    g.splits = (ng + g.kbs - 1) / g.kbs;
    g.ws = g.splits > 1 ? (size_t)g.tiles * g.splits * (32 * g.mt) * GBN * 4 : 0;
    return g;
}

}  // namespace

size_t gemm_workspace_bytes(int type, int64_t m, int64_t n, int64_t k) {
    if (type != TYPE_Q4_K || m <= 0 || n <= 0 || k <= 0 || k % QK_K) return (size_t)-1;
    const GemmPlan g = gemm_plan(m, n, k);
    if (g.tiles > GEMM_MAX_TILES) return (size_t)-1;
    return g.ws;
}

hipError_t launch_gemm(const WLayout &w, int64_t n, int64_t k, const ActPlanes &x, int64_t m, float *y, int32_t *S,
                       int32_t *Smin, void *ws, size_t ws_bytes, int *counters, hipStream_t s) {
    if (w.type != TYPE_Q4_K) return hipErrorNotSupported;
    if (!w.slab || !y || !x.qs || !x.d || !x.bsum16 || m <= 0 || n <= 0 || k <= 0 || k % QK_K) return hipErrorInvalidValue;
    if (m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff || w.ng != k / QK_K) return hipErrorInvalidValue;
    if ((S == nullptr) != (Smin == nullptr)) return hipErrorInvalidValue;
    const GemmPlan g = gemm_plan(m, n, k);
    if (g.tiles > GEMM_MAX_TILES) return hipErrorNotSupported;
    if (g.splits > 1 && (!ws || ws_bytes < g.ws || !counters)) return hipErrorInvalidValue;
    GemmParams p;
    p.w = w.slab;
    p.rb_stride = w.rb_stride;
    p.ng = w.ng;
    p.xq = x.qs;
    p.xd = x.d;
    p.xbs = x.bsum16;
    p.y = y;
    p.m = (int)m;
    p.n = (int)n;
    p.k = (int)k;
    p.ntm = g.ntm;
    p.tiles = g.tiles;
    p.splits = g.splits;
    p.kbs = g.kbs;
    p.items = g.tiles * g.splits;
    p.per_xcd = (p.items + NXCD - 1) / NXCD;
    p.part = (float *)ws;
    p.counters = counters;
    p.S = S;
    p.Smin = Smin;
    const unsigned grid = (unsigned)(p.per_xcd * NXCD);
    if (g.mt == 4) {
        if (S) gemm_q4k_kernel<4, true><<<grid, 256, 0, s>>>(p);
        else gemm_q4k_kernel<4, false><<<grid, 256, 0, s>>>(p);
    } else {
        if (S) gemm_q4k_kernel<2, true><<<grid, 256, 0, s>>>(p);
        else gemm_q4k_kernel<2, false><<<grid, 256, 0, s>>>(p);
    }
    return hipGetLastError();
}

}  // namespace aq
