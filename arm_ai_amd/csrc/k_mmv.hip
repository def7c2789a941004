// k_mmv.hip -- matvec of a few batch rows (8 per launch) on the int8 matrix
// cores, Q4_K and Q6_K weights against Q8_K activations, gfx950.
//
// Replaces the column loop of candle-core 0.8.4 k_quants::matmul<T> (each
// output = T::vec_dot(k, W[col], xq[row])) for a batch of a few rows, as at
// native/arm_ai_nif/src/llama_candle.rs:119 when several sequences decode
// together.  The integer parts (S = sum_j sc_j * isum_j, Smin) are exact; the
// f32 combination is the one-row kernel's: per super-block
// y += (d_w*d_x)*S - (dmin_w*d_x)*Smin (Q4_K), y += (d_w*d_x)*S (Q6_K).
//
// A 16 x 16 MFMA tile is 16 weight rows (the columns of the product) by 16
// "batch" rows made of the 8 activation rows twice: rows 0..7 are the
// activation rows restricted to one sub-block s and rows 8..15 the same rows
// restricted to the next sub-block s'.  The K slots of the weight operand
// hold elements of s and of s'; each activation row is zero in the slots of
// the other sub-block.
//   * Q4_K: s, s' = 2c, 2c+1 (32 elements each), v_mfma_i32_16x16x64_i8,
//     four per super-block.  Lane (i, j) = (lane%16, lane/16) loads 8 qs
//     bytes of its weight row, qs[32c + 8j..]: their low nibbles fill K slots
//     0..7 (elements of 2c), their high nibbles slots 8..15 (elements of
//     2c+1).  Its activation row i%8 fills slots 0..7 (i < 8) or 8..15.
//   * Q6_K: s, s' = 2p, 2p+1 (16 elements each), v_mfma_i32_16x16x32_i8,
//     eight per super-block.  Lane groups j = 0, 1 hold elements of 2p, 2, 3
//     of 2p+1; the activation lanes of the other sub-block are masked to zero.
// One MFMA thus gives isum of sub-block s (output rows 0..7, lanes 0..31) and
// of s' (rows 8..15, lanes 32..63); each lane applies its own sub-block's
// scale with an integer multiply-add, and the two halves are added at the
// end of the super-block.  The min term (Q4_K: sum_g bsums[g]*m[g/2]) and
// the Q6_K offset term (sum_j sc_j*bsums[j], the -32 of q6) are one
// v_mfma_f32_16x16x16_f16 per super-block: bsums (|.| <= 2048), 6-bit mins and
// int8 scales are exact in f16 and every partial sum is below 2^24, so both
// are exact.
//
// The quantised activation of the pass (8 rows) is copied once per
// workgroup into LDS by buffer-to-LDS loads (no registers; each instruction
// moves 8 rows x 128 contiguous bytes), interleaving the rows so that every
// MFMA operand read is one conflict-free ds_read_b64: per super-block,
// 16-element piece P of row b sits at (P*8 + b)*16.  (Reading it from the
// cache inside the loop instead cost more than the weight stream: every
// wavefront re-requested the same lines.)  Only the weights are streamed,
// from the row-block tiles (each load instruction reads whole 128-byte
// lines), in a ring of register stages per wavefront.
//
// A wavefront owns one 16-row tile and a chunk of its super-blocks (every
// kch-th one); the wavefronts of a tile's chunks are in one workgroup and add
// their partials in chunk order through LDS (deterministic).  Workgroups stay resident and
// loop over the (tiles x chunks) iterations, so each fills its LDS once.
// Q4_K rows of more than 8 quads (4 super-blocks each) are split into K
// parts: a workgroup holds one part's activation and takes tiles of that
// part only (the grid is a multiple of the part count), writes the part's
// sums to a workspace, and mmv_reduce_kernel adds the parts in order.
#include "aq_internal.h"

#include <algorithm>
#include <mutex>

namespace aq {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int TILE = 16;         // weight rows per wavefront tile
constexpr int MAXB = 8;          // activation rows per launch
constexpr int MAX_WAVES = 8;     // wavefronts per workgroup
constexpr int TARGET_WAVES = 4096;
constexpr int MIN_GPC = 2;       // super-blocks per chunk, at least (when there are that many)
// Q6_K: weight stages per wavefront (loads issued NS - 1 steps ahead; a stage
// is 17 registers) and the vector memory instructions of one stage (load_w)
template <int TYPE>
constexpr int stages_of() { return 3; }
template <int TYPE>
constexpr int loads_of() { return 8; }
// LDS of the pass's activation: qs [ng][16 pieces][8 rows][16 B], f16 bsums
// [ng][2 pieces][8 rows][16 B] (padded to whole copies of 4 super-blocks),
// d [ng][8 rows] f32 (padded to whole copies of 8 super-blocks), then the
// reduction slots [waves][8 rows][16] f32.
constexpr int LQ = 2048;  // qs bytes per super-block
constexpr int LB = 256;   // bsums bytes per super-block
constexpr int LD = 32;    // d bytes per super-block
constexpr int LRED = MAXB * TILE * 4;  // reduction bytes per wavefront
constexpr size_t LDS_CAP = 160 * 1024;
constexpr int LZ = 2048;  // a zero block: operand reads of inactive lanes
struct ActLds {
    int bs, d, zero, red, bytes;  // offsets
};
__host__ __device__ inline ActLds act_lds(int ng, int nw) {
    ActLds a;
    a.bs = ng * LQ;
    a.d = a.bs + (ng + 3) / 4 * 4 * LB;
    a.zero = a.d + (ng + 7) / 8 * 8 * LD;
    a.red = a.zero + LZ;
    a.bytes = a.red + nw * LRED;
    return a;
}

struct MmvParams {
    const uint8_t *w;    // row-block tiles
    const uint16_t *wd;  // Q6_K d plane
    int64_t rb_stride;
    int n, k, ng, nrb, m;
    int tiles, kch, gpc, tpw, iters;  // an iteration: tpw tiles x kch chunks, one wavefront each
    int ks, qpp;                      // Q4_K: K parts of qpp quads (iterations: tile groups x parts)
    float *part;                      // ks > 1: the parts' sums [ks][m][n], added by mmv_reduce_kernel
    const int8_t *qs;                 // [m][k]
    const float *d;                   // [m][k/256]
    const uint16_t *bs16;             // [m][k/16] f16 bsums
    float *y;                         // [m][n]
    int32_t *S, *Smin;                // [m][n][ng] or null
};

template <int TYPE>
struct WStage;
template <>
struct WStage<TYPE_Q6_K> {
    u32x2 ql[2][2], qh[2];  // [hh][A/B] 8 bytes of ql pieces 4hh + t (+2), qh piece 8 + 2hh + t
    u32x4 sc;               // piece 12: int8 scales[16]
    uint32_t d;             // f16 bits
};

struct Lane {
    int lane, i, j, h;  // i = lane % 16, j = lane / 16, h = lane / 32
};

// Weights of super-block g of this wavefront's tile (the tile's two row
// blocks are one descriptor; lanes 8..15 take the second).
template <int TYPE>
__device__ __forceinline__ void load_w(WStage<TYPE> &W, const MmvParams &p, const rsrc_t &rw, const rsrc_t &rwd,
                                       int g, bool g_ok, const Lane &L) {
    const uint32_t row_off = (uint32_t)((L.i >> 3) * p.rb_stride) + (uint32_t)((L.i & 7) * 16);
    {
        const uint32_t base = g_ok ? row_off + (uint32_t)(g * 13 * 128) + 8 * (L.j & 1) : BUF_OOB;
        const int t = L.j >> 1;
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            W.ql[hh][0] = __builtin_amdgcn_raw_buffer_load_b64(rw, base + (4 * hh + t) * 128, 0, BUF_NT);
            W.ql[hh][1] = __builtin_amdgcn_raw_buffer_load_b64(rw, base + (4 * hh + 2 + t) * 128, 0, BUF_NT);
            W.qh[hh] = __builtin_amdgcn_raw_buffer_load_b64(rw, base + (8 + 2 * hh + t) * 128, 0, BUF_NT);
        }
        W.sc = __builtin_amdgcn_raw_buffer_load_b128(rw, g_ok ? row_off + (uint32_t)((g * 13 + 12) * 128) : BUF_OOB, 0,
                                                     BUF_NT);
        W.d = __builtin_amdgcn_raw_buffer_load_b16(
            rwd, g_ok ? (uint32_t)((((L.i >> 3) * p.ng + g) * RB + (L.i & 7)) * 2) : BUF_OOB, 0, BUF_NT);
    }
}

// The pass's activation into LDS, super-blocks g0 .. g0 + ngk - 1, issued
// by every wavefront (copy q of a region goes to LDS q * 1024 (256 for d);
// lane l takes row l%8 and piece l/8 of the copy; super-block g0 + i lands
// at entry i).  Rows past m read zeros; the copies past the last super-block
// land in the regions' padding.  ZERO: also clear the zero block.  Waited
// for by the caller (vmcnt for the copies, lgkmcnt for the clearing).
template <bool ZERO>
__device__ __forceinline__ void fill_act(uint8_t *lds, const MmvParams &p, const ActLds &a, int g0, int ngk, int wave,
                                         int nw, int lane) {
    const int b = lane & 7, pc = lane >> 3;
    const rsrc_t rq = buf_rsrc(p.qs, (uint32_t)(p.m * p.k));
    const uint32_t vq = (uint32_t)(b * p.k + g0 * QK_K + 16 * pc);
    for (int q = wave; q < 2 * ngk; q += nw) buf_to_lds16(rq, lds + q * 1024, vq + 128 * q, 0);
    const rsrc_t rbs = buf_rsrc(p.bs16, (uint32_t)(p.m * (p.k / 16) * 2));
    const uint32_t vb = (uint32_t)(b * (p.k / 8) + g0 * 32 + 16 * pc);
    for (int q = wave; q < (ngk + 3) / 4; q += nw) buf_to_lds16(rbs, lds + a.bs + q * 1024, vb + 128 * q, 0);
    const rsrc_t rd = buf_rsrc(p.d, (uint32_t)(p.m * p.ng * 4));
    const uint32_t vd = (uint32_t)((b * p.ng + g0 + pc) * 4);
    for (int q = wave; q < (ngk + 7) / 8; q += nw) buf_to_lds4(rd, lds + a.d + q * 256, vd + 32 * q, 0);
    if (ZERO)
        for (int t = 64 * wave + lane; t < LZ / 16; t += 64 * nw) *(u32x4 *)(lds + a.zero + 16 * t) = u32x4{0u, 0u, 0u, 0u};
}

__device__ __forceinline__ long as_long(const u32x2 u) { return (long)(((uint64_t)u.y << 32) | (uint64_t)u.x); }
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    const _Float16 ha = (_Float16)a, hb = (_Float16)b;
    return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}
__device__ __forceinline__ v4h as_v4h(uint32_t lo, uint32_t hi) { return __builtin_bit_cast(v4h, u32x2{lo, hi}); }
__device__ __forceinline__ int ubyte(uint32_t w, int sh) { return (int)((w >> sh) & 0xffu); }
__device__ __forceinline__ int sbyte(uint32_t w, int sh) { return (int)(int8_t)(w >> sh); }

// One Q6_K super-block of a tile: adds its integer sums into S (this lane's
// sub-blocks) and returns the f16-MFMA offset term sum sc*bsums.
// la, lb: the super-block's LDS quants and bsums.
template <int TYPE>
__device__ __forceinline__ v4f superblock(const WStage<TYPE> &W, const uint8_t *la, const uint8_t *lb, const Lane &L,
                                          int S[4]) {
    const v4i z = {0, 0, 0, 0};
    const v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
    // bsums 4j..4j+3 of row i%8: piece j/2, half j%2
    const u32x2 bs = *(const u32x2 *)(lb + ((L.j >> 1) * MAXB + (L.i & 7)) * 16 + 8 * (L.j & 1));
    {
        const uint32_t scw[4] = {W.sc.x, W.sc.y, W.sc.z, W.sc.w};
        // activation elements 32p + 8j.. of row i%8 (piece 2p + j/2, half j%2), zero unless
        // lane group j carries this row half's sub-block
        const uint8_t *aq = la + ((L.j >> 1) * MAXB + (L.i & 7)) * 16 + 8 * (L.j & 1);
        const uint32_t keep = (L.i < 8) == (L.j < 2) ? 0xFFFFFFFFu : 0u;
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const u32x2 a = W.ql[hh][0], bq = W.ql[hh][1], hq = W.qh[hh];
            const uint32_t av[2] = {a.x, a.y}, bv[2] = {bq.x, bq.y}, hv[2] = {hq.x, hq.y};
#pragma unroll
            for (int gq = 0; gq < 4; gq++) {
                uint32_t qv[2];
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const uint32_t src = gq & 1 ? bv[e] : av[e];
                    const uint32_t lo = gq < 2 ? src & 0x0F0F0F0Fu : (src >> 4) & 0x0F0F0F0Fu;
                    qv[e] = lo | (((hv[e] >> (2 * gq)) & 0x03030303u) << 4);
                }
                const int pi = 4 * hh + gq;  // sub-blocks 2pi (lanes 0..31) and 2pi + 1 (lanes 32..63)
                const u32x2 x = *(const u32x2 *)(aq + pi * 2 * MAXB * 16);
                const v4i acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(u32x2{x.x & keep, x.y & keep}),
                                                                      as_long(u32x2{qv[0], qv[1]}), z, 0, 0, 0);
                const int sc = sbyte(scw[pi >> 1], 8 * (2 * (pi & 1) + L.h));
                // |acc| <= 16 * 63 * 128 and |sc| <= 128 fit 24 bits: the
                // full-rate 24-bit multiply gives the same integers
                S[0] += __mul24(sc, acc.x);
                S[1] += __mul24(sc, acc.y);
                S[2] += __mul24(sc, acc.z);
                S[3] += __mul24(sc, acc.w);
            }
        }
        // offset term: K slot 4j + t is bsums[4j + t] against scale 4j + t
        const uint32_t w = scw[L.j];
        const v4h bsc = as_v4h(pack_h2((float)sbyte(w, 0), (float)sbyte(w, 8)),
                               pack_h2((float)sbyte(w, 16), (float)sbyte(w, 24)));
        return __builtin_amdgcn_mfma_f32_16x16x16f16(as_v4h(bs.x, bs.y), bsc, zf, 0, 0, 0);
    }
}

template <int TYPE, bool DUMP>
__global__ __launch_bounds__(MAX_WAVES * 64) void mmv_kernel(MmvParams p) {
    static_assert(TYPE == TYPE_Q6_K, "Q4_K has its own kernel");
    extern __shared__ __align__(16) uint8_t lds[];
    Lane L;
    L.lane = threadIdx.x & 63;
    L.i = L.lane & 15;
    L.j = L.lane >> 4;
    L.h = L.lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int tw = wave / p.kch, chunk = wave - tw * p.kch;
    // chunk c takes super-blocks c, c + kch, ...: at each step the wavefronts
    // of a tile read neighbouring super-blocks (longer runs of DRAM)
    const int nmine = chunk < p.ng ? (p.ng - chunk + p.kch - 1) / p.kch : 0;
    auto gsb = [&](int s) { return chunk + s * p.kch; };
    const int nw = p.tpw * p.kch;
    const ActLds al = act_lds(p.ng, nw);
    float *red = (float *)(lds + al.red);  // [wave][b][tile row]
    const float *ldx = (const float *)(lds + al.d);

    // Per-iteration state of this wavefront: its tile, its super-block count
    // and the tile's weight descriptors.
    constexpr int NS = stages_of<TYPE>();
    int tile = 0, cnt = 0;
    rsrc_t rw, rwd;
    WStage<TYPE> ws[NS];
    auto begin = [&](int it) {  // set up iteration it and issue its first NS - 1 weight stages
        tile = it * p.tpw + tw;
        cnt = it < p.iters && tile < p.tiles ? nmine : 0;  // wave-uniform
        const int rb0 = 2 * tile;
        const int nrb_t = cnt > 0 ? min(2, p.nrb - rb0) : 0;
        rw = buf_rsrc(p.w + (cnt > 0 ? (int64_t)rb0 * p.rb_stride : 0), (uint32_t)(nrb_t * p.rb_stride));
        rwd = buf_rsrc(TYPE == TYPE_Q6_K && cnt > 0 ? p.wd + (int64_t)rb0 * p.ng * RB : p.wd,
                       TYPE == TYPE_Q6_K ? (uint32_t)(nrb_t * p.ng * RB * 2) : 0u);
#pragma unroll
        for (int u = 0; u < NS - 1; u++) load_w<TYPE>(ws[u], p, rw, rwd, gsb(u), u < cnt, L);
    };

    // the activation copies first, then the first weight stages: waiting for
    // the copies (vmcnt down to the weight loads) leaves the weights in flight
    fill_act<false>(lds, p, al, 0, p.ng, wave, nw, L.lane);
    __builtin_amdgcn_sched_barrier(0);
    begin(blockIdx.x);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<(NS - 1) * loads_of<TYPE>()>();
    stage_barrier();

    const rsrc_t ry = buf_rsrc(p.y, (uint32_t)(p.m * p.n * 4));
    for (int it = blockIdx.x; it < p.iters; it += gridDim.x) {  // workgroup-uniform
        const int row = tile * TILE + L.i;  // output column of this lane
        float f[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        auto step = [&](const WStage<TYPE> &W, int g) {
            int S[4] = {0, 0, 0, 0};
            const v4f t = superblock<TYPE>(W, lds + g * LQ, lds + al.bs + g * LB, L, S);
            // lanes 0..31 hold batch rows 4j + r of sub-blocks s, lanes 32..63 of s'
#pragma unroll
            for (int r = 0; r < 4; r++) S[r] += __shfl_xor(S[r], 32);
            const int tv[4] = {(int)t.x, (int)t.y, (int)t.z, (int)t.w};
            const v4f dx = *(const v4f *)(ldx + g * MAXB + 4 * (L.j & 1));
            const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
            const float dw = f16_bits_to_f32(W.d);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                S[r] -= 32 * tv[r];  // q6 - 32: sum sc*(isum - 32*bsum)
                f[r] += (dw * dxv[r]) * (float)S[r];
            }
            if (DUMP) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int b = 4 * L.j + r;
                    if (L.lane < 32 && b < p.m && row < p.n) {
                        const int64_t o = ((int64_t)b * p.n + row) * p.ng + g;
                        p.S[o] = S[r];
                        p.Smin[o] = 0;
                    }
                }
            }
        };
        // ring: stage u % NS holds step u; the loads of step u + NS - 1 are
        // issued before step u is computed (past the chunk they read zeros).
        // Every path issues the same loads -- only the compute is skipped --
        // so the compiler's s_waitcnt counts stay exact (a branch around a
        // load makes it wait for all of them).
        for (int s = 0; s < cnt; s += NS) {
#pragma unroll
            for (int u = 0; u < NS; u++) {
                load_w<TYPE>(ws[(u + NS - 1) % NS], p, rw, rwd, gsb(s + u + NS - 1), s + u + NS - 1 < cnt, L);
                if (s + u < cnt) step(ws[u], gsb(s + u));
            }
        }
        begin(it + gridDim.x);  // the next iteration's first loads overlap this one's stores

        if (p.kch == 1) {  // workgroup-uniform
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int b = 4 * L.j + r;
                const bool ok = L.lane < 32 && b < p.m && row < p.n;
                __builtin_amdgcn_raw_buffer_store_b32(f32_as_u32(f[r]), ry, ok ? (uint32_t)((b * p.n + row) * 4) : BUF_OOB,
                                                      0, 0);
            }
            continue;
        }
        if (L.lane < 32) {
#pragma unroll
            for (int r = 0; r < 4; r++) red[(wave * MAXB + 4 * L.j + r) * TILE + L.i] = f[r];
        }
        lds_barrier();
        if (chunk == 0) {  // wave-uniform: the tile's first wavefront adds the chunks in order
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int b = 4 * L.j + r;
                float s = 0.0f;
                for (int c = 0; c < p.kch; c++) s += red[((wave + c) * MAXB + (b & 7)) * TILE + L.i];
                const bool ok = L.lane < 32 && b < p.m && row < p.n;
                __builtin_amdgcn_raw_buffer_store_b32(f32_as_u32(s), ry, ok ? (uint32_t)((b * p.n + row) * 4) : BUF_OOB, 0,
                                                      0);
            }
        }
        lds_barrier();  // red is rewritten by the next iteration
    }
}

// ---------------------------------------------------------------- Q4_K
// Lane (n, j) = (lane%16, lane/16) streams whole super-blocks: super-block
// 4q + j of row n of the tile (9 b128 loads per step, 16 rows x 4
// super-blocks = two row blocks x 4 groups, whole 128-byte lines).  Each
// v_mfma_i32_16x16x64_i8 then works on all four lane groups at once, each on
// its own super-block: output rows 4j..4j+3 take only lane group j's K slots
// (the activation operand of lane (i, j) is zero unless j = i/4; those lanes
// read the LDS zero block), so lane (n, j) receives the 16-element sums of
// its own super-block for 4 batch rows.  The 16 slots of one MFMA are the low
// (or high) nibbles of one qs piece: 16 elements of one sub-block; the two
// pieces of a sub-block accumulate in one MFMA chain, whose result the lane
// scales by the sub-block's 6-bit scale with an integer multiply-add.  Per
// step: 8 sub-blocks x 2 pieces x 2 batch halves = 32 MFMAs for 4
// super-blocks, and the min term on v_mfma_f32_16x16x32_f16 (8 bsums per
// lane group).
template <bool DUMP>
__global__ __launch_bounds__(512) void mmv_q4k_kernel(MmvParams p) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63, n = lane & 15, j = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int nw = p.tpw * p.kch;
    const int tw = wave / p.kch, chunk = wave - tw * p.kch;
    // K part kp of this workgroup (the grid is a multiple of ks, so every
    // iteration of the workgroup is in the same part): quads q0 .. q0 + nqk - 1
    const int kp = (int)blockIdx.x % p.ks;
    const int q0 = kp * p.qpp, nq = (p.ng + 3) / 4;
    const int nqk = min(p.qpp, nq - q0), g0 = 4 * q0;
    const ActLds al = act_lds(4 * p.qpp, nw);
    float *red = (float *)(lds + al.red);  // [wave][b][tile row]
    // chunk c takes quads (4 super-blocks) q0 + c, q0 + c + kch, ...
    const int nmine = chunk < nqk ? (nqk - chunk + p.kch - 1) / p.kch : 0;

    int tile = 0, cnt = 0;
    rsrc_t rw;
    u32x4 wa[9], wb[9];
    auto load = [&](u32x4 (&W)[9], int s) {
        const int g = 4 * (q0 + chunk + s * p.kch) + j;
        const uint32_t off = g < p.ng ? (uint32_t)((n >> 3) * p.rb_stride + g * 9 * 128 + (n & 7) * 16) : BUF_OOB;
#pragma unroll
        for (int i = 0; i < 9; i++) W[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, off + i * 128, 0, BUF_NT);
    };
    auto begin = [&](int it) {  // set up iteration it and issue its first step's loads
        tile = it / p.ks * p.tpw + tw;
        cnt = it < p.iters && tile < p.tiles ? nmine : 0;  // wave-uniform
        const int rb0 = 2 * tile;
        const int nrb_t = cnt > 0 ? min(2, p.nrb - rb0) : 0;
        rw = buf_rsrc(p.w + (cnt > 0 ? (int64_t)rb0 * p.rb_stride : 0), (uint32_t)(nrb_t * p.rb_stride));
        load(wa, 0);
    };

    // the activation copies first, then the first weight loads: waiting for
    // the copies (vmcnt down to the 9 weight loads) leaves the weights in flight
    fill_act<true>(lds, p, al, g0, 4 * nqk, wave, nw, lane);
    __builtin_amdgcn_sched_barrier(0);
    begin(blockIdx.x);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<9>();
    lds_barrier();

    const rsrc_t ry = buf_rsrc(p.ks > 1 ? p.part + (int64_t)kp * p.m * p.n : p.y, (uint32_t)(p.m * p.n * 4));
    const v4i z = {0, 0, 0, 0};
    const v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int it = blockIdx.x; it < p.iters; it += gridDim.x) {  // workgroup-uniform
        const int row = tile * TILE + n;
        float f[2][4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};  // [batch half][r]: batch row 4h + r
        auto step = [&](const u32x4 (&W)[9], int s) {
            const int g = 4 * (q0 + chunk + s * p.kch) + j;  // this lane group's super-block
            const bool g_ok = g < p.ng;
            const int gl = g_ok ? g - g0 : 0;  // its LDS entry
            // activation operand of lane (i = n, j): row 4h + n%4 of super-block g when j = n/4
            const bool act = g_ok && j == (n >> 2);
            const int ab = act ? gl * LQ + (n & 3) * 16 : al.zero;  // + 64 for batch half 1 (zero block: stays zero)
            const int bb = act ? al.bs + gl * LB + (n & 3) * 16 : al.zero;
            const uint32_t u0 = W[0].y, u1 = W[0].z, u2 = W[0].w;
            // candle's utmp form of GGML get_scale_min_k4 (6-bit scales and mins)
            const uint32_t sc03 = u0 & 0x3F3F3F3Fu;
            const uint32_t sc47 = (u2 & 0x0F0F0F0Fu) | (((u0 >> 6) & 0x03030303u) << 4);
            const uint32_t mn03 = u1 & 0x3F3F3F3Fu;
            const uint32_t mn47 = ((u2 >> 4) & 0x0F0F0F0Fu) | (((u1 >> 6) & 0x03030303u) << 4);
            int S[2][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
            for (int sb = 0; sb < 8; sb++) {  // sub-block sb = 2c + hl
                // keeps the scheduler from hoisting every activation read of the
                // super-block ahead (their registers would spill)
                __builtin_amdgcn_sched_barrier(0);
                const int c = sb >> 1, hl = sb & 1;
                const int sc = ubyte(c < 2 ? sc03 : sc47, 8 * (2 * (c & 1) + hl));
                v4i acc[2] = {z, z};
#pragma unroll
                for (int half = 0; half < 2; half++) {
                    // piece 1 + 2c + half = qs[32c + 16half..]: its low nibbles are elements
                    // 16half + t of sub-block 2c, its high nibbles the same of 2c + 1
                    const u32x4 pc = W[1 + 2 * c + half];
                    v4i wq;
                    wq.x = (int)((pc.x >> (4 * hl)) & 0x0F0F0F0Fu);
                    wq.y = (int)((pc.y >> (4 * hl)) & 0x0F0F0F0Fu);
                    wq.z = (int)((pc.z >> (4 * hl)) & 0x0F0F0F0Fu);
                    wq.w = (int)((pc.w >> (4 * hl)) & 0x0F0F0F0Fu);
                    const int P = 2 * sb + half;  // activation piece (16 elements) = 4c + 2hl + half
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const v4i a = *(const v4i *)(lds + ab + (act ? 64 * h : 0) + P * MAXB * 16);
                        acc[h] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, wq, acc[h], 0, 0, 0);
                    }
                }
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    // |acc| <= 32 * 15 * 128 and sc <= 63 fit 24 bits: the
                    // full-rate 24-bit multiply gives the same integers
                    S[h][0] += __mul24(sc, acc[h].x);
                    S[h][1] += __mul24(sc, acc[h].y);
                    S[h][2] += __mul24(sc, acc[h].z);
                    S[h][3] += __mul24(sc, acc[h].w);
                }
            }
            // min term: K slot 8u + t is bsums[8u + t] of sub-block 4u + t/2
            v4h bmh[2][2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const uint32_t mw = u ? mn47 : mn03;
                const float m0 = (float)ubyte(mw, 0), m1 = (float)ubyte(mw, 8), m2 = (float)ubyte(mw, 16),
                            m3 = (float)ubyte(mw, 24);
                bmh[u][0] = as_v4h(pack_h2(m0, m0), pack_h2(m1, m1));
                bmh[u][1] = as_v4h(pack_h2(m2, m2), pack_h2(m3, m3));
            }
            const float dw = f16_bits_to_f32(W[0].x), dmw = f16_bits_to_f32(W[0].x >> 16);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                v4f sm = zf;
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const u32x4 bv = *(const u32x4 *)(lds + bb + (act ? 64 * h + u * MAXB * 16 : 0));
                    const v8h a = __builtin_bit_cast(v8h, bv);
                    const v8h bm = __builtin_shufflevector(bmh[u][0], bmh[u][1], 0, 1, 2, 3, 4, 5, 6, 7);
                    sm = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bm, sm, 0, 0, 0);
                }
                const v4f dx = *(const v4f *)(lds + al.d + gl * LD + 16 * h);
                const float dxv[4] = {dx.x, dx.y, dx.z, dx.w}, smv[4] = {sm.x, sm.y, sm.z, sm.w};
#pragma unroll
                for (int r = 0; r < 4; r++) f[h][r] += (dw * dxv[r]) * (float)S[h][r] - (dmw * dxv[r]) * smv[r];
                if (DUMP) {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int b = 4 * h + r;
                        if (g_ok && b < p.m && row < p.n) {
                            const int64_t o = ((int64_t)b * p.n + row) * p.ng + g;
                            p.S[o] = S[h][r];
                            p.Smin[o] = (int)smv[r];
                        }
                    }
                }
            }
        };
        // two-stage ping-pong; the tail is peeled so that no load is issued
        // past the chunk and every load is unconditional within its block
        // (a branch around a load makes the compiler wait for all of them)
        int s = 0;
        for (; s + 2 < cnt; s += 2) {
            load(wb, s + 1);
            step(wa, s);
            load(wa, s + 2);
            step(wb, s + 1);
        }
        if (cnt - s == 2) {
            load(wb, s + 1);
            step(wa, s);
            step(wb, s + 1);
        } else if (cnt - s == 1) {
            step(wa, s);
        }
        // add the four lane groups' super-blocks: lanes 0..15 hold the chunk's sum
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                f[h][r] += __shfl_xor(f[h][r], 16);
                f[h][r] += __shfl_xor(f[h][r], 32);
            }
        begin(it + gridDim.x);  // the next iteration's first loads overlap this one's stores

        if (p.kch == 1) {  // workgroup-uniform
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int b = 4 * h + r;
                    const bool ok = lane < 16 && b < p.m && row < p.n;
                    __builtin_amdgcn_raw_buffer_store_b32(f32_as_u32(f[h][r]), ry,
                                                          ok ? (uint32_t)((b * p.n + row) * 4) : BUF_OOB, 0, 0);
                }
            continue;
        }
        if (lane < 16) {
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int r = 0; r < 4; r++) red[(wave * MAXB + 4 * h + r) * TILE + n] = f[h][r];
        }
        lds_barrier();
        if (chunk == 0) {  // wave-uniform: the tile's first wavefront adds the chunks in order
#pragma unroll
            for (int b = 0; b < MAXB; b++) {
                float acc = 0.0f;
                for (int c = 0; c < p.kch; c++) acc += red[((wave + c) * MAXB + b) * TILE + n];
                const bool ok = lane < 16 && b < p.m && row < p.n;
                __builtin_amdgcn_raw_buffer_store_b32(f32_as_u32(acc), ry, ok ? (uint32_t)((b * p.n + row) * 4) : BUF_OOB,
                                                      0, 0);
            }
        }
        lds_barrier();  // red is rewritten by the next iteration
    }
}

// y[i] = sum over the K parts of part[kp][i], in part order (one output per thread)
__global__ __launch_bounds__(256) void mmv_reduce_kernel(const float *__restrict__ part, int ks, int mn,
                                                         float *__restrict__ y) {
    const int i = (int)blockIdx.x * 256 + (int)threadIdx.x;
    if (i >= mn) return;
    float t = part[i];
    for (int kp = 1; kp < ks; kp++) t += part[(int64_t)kp * mn + i];
    y[i] = t;
}

int cu_count() {
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (!cached[dev]) {
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        cached[dev] = c;
    }
    return cached[dev];
}

// Dynamic LDS above 64 KB has to be allowed per kernel, once.
template <void (*F)(MmvParams)>
hipError_t allow_lds() {
    static std::once_flag once;
    static hipError_t err = hipSuccess;
    std::call_once(once, [] {
        err = hipFuncSetAttribute((const void *)F, hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_CAP);
    });
    return err;
}

// ng_lds: the super-blocks of activation a workgroup holds in LDS (the
// whole row, or a Q4_K K part)
template <void (*F)(MmvParams)>
hipError_t launch_f(MmvParams p, int ng_lds, int64_t m, const ActPlanes &act, float *y, int32_t *S, int32_t *Smin,
                    void *ws, size_t ws_bytes, hipStream_t s) {
    const int nw = p.tpw * p.kch;
    const size_t lds = (size_t)act_lds(ng_lds, nw).bytes;
    if (lds > LDS_CAP) return hipErrorNotSupported;
    if (p.ks < 1 || p.iters % p.ks) return hipErrorInvalidValue;
    if (p.ks > 1 && (!ws || ws_bytes < (size_t)p.ks * MAXB * p.n * 4)) return hipErrorInvalidValue;
    p.part = p.ks > 1 ? (float *)ws : nullptr;
    hipError_t e = allow_lds<F>();
    if (e != hipSuccess) return e;
    int per_cu = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)F, nw * 64, lds);
    if (e != hipSuccess) return e;
    const int cus = cu_count();
    if (per_cu <= 0 || cus <= 0) return hipErrorNotSupported;
    // a multiple of ks workgroups, so that each stays in one K part
    int64_t g = std::min((int64_t)p.iters, (int64_t)per_cu * cus);
    g = std::max<int64_t>(p.ks, g / p.ks * p.ks);
    const unsigned grid = (unsigned)g;
    // passes of up to MAXB rows; every plane is row-major, so a pass is an offset
    for (int64_t r0 = 0; r0 < m; r0 += MAXB) {
        p.m = (int)(m - r0 < MAXB ? m - r0 : MAXB);
        p.qs = act.qs + r0 * p.k;
        p.d = act.d + r0 * p.ng;
        p.bs16 = act.bsum16 + r0 * (p.k / 16);
        p.y = y + r0 * p.n;
        p.S = S ? S + r0 * p.n * p.ng : nullptr;
        p.Smin = Smin ? Smin + r0 * p.n * p.ng : nullptr;
        F<<<grid, dim3(nw * 64), lds, s>>>(p);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (p.ks > 1) {
            const int mn = p.m * p.n;
            mmv_reduce_kernel<<<(unsigned)((mn + 255) / 256), 256, 0, s>>>(p.part, p.ks, mn, p.y);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

// The Q4_K launch shape: kch chunks per tile, tpw tiles per workgroup, ks K
// parts (quads split as evenly as whole quads allow)
struct Q4kShape {
    int kch, tpw, ks;
};
Q4kShape q4k_shape(int tiles, int ng) {
    // quads of 4 super-blocks per step; chunks of at least 3 quads when
    // there are that many, about 2048 wavefronts in all, up to 8 per
    // workgroup (a wavefront streams a few steps of 9.2 KB with two in
    // flight, which keeps HBM busy at a few wavefronts per CU)
    const int nq = (ng + 3) / 4;
    const int64_t want = (2048 + tiles - 1) / tiles;
    Q4kShape q;
    q.kch = (int)std::min<int64_t>(want, std::min(8, std::max(1, nq / 3)));
    q.tpw = std::max(1, 4 / q.kch);
    q.ks = 1;
    if (nq > 8) {
        // long rows: every workgroup copies the activation of its K range
        // into LDS, which for a whole row (8 rows x k bytes of quants) is as
        // many bytes as a tile's weights.  K parts of 4 quads, one wavefront
        // per tile and 4 tiles per workgroup: 4096 x 14336 at batch 8 took
        // 11.8-12.0 us with the parts' reduce launch against 13.0 us whole
        // (3 and 7 parts, 2-8 tiles and 2 chunks per tile measured slower)
        q.ks = (nq + 3) / 4;
        q.kch = 1;
        q.tpw = 4;
    }
    return q;
}

hipError_t launch_q4k(MmvParams p, Q4kShape q, int64_t m, const ActPlanes &act, float *y, int32_t *S, int32_t *Smin,
                      void *ws, size_t ws_bytes, hipStream_t s) {
    const int nq = (p.ng + 3) / 4;
    if (q.kch < 1 || q.tpw < 1 || q.kch * q.tpw > MAX_WAVES || q.ks < 1 || q.ks > nq) return hipErrorInvalidValue;
    p.qpp = (nq + q.ks - 1) / q.ks;
    p.ks = (nq + p.qpp - 1) / p.qpp;  // every part holds a quad
    p.kch = std::min(q.kch, p.qpp);
    p.tpw = q.tpw;
    p.gpc = 0;
    p.iters = (p.tiles + p.tpw - 1) / p.tpw * p.ks;
    return S ? launch_f<mmv_q4k_kernel<true>>(p, 4 * p.qpp, m, act, y, S, Smin, ws, ws_bytes, s)
             : launch_f<mmv_q4k_kernel<false>>(p, 4 * p.qpp, m, act, y, S, Smin, ws, ws_bytes, s);
}

bool mmv_args_ok(const WLayout &w, int64_t n, int64_t k) {
    return (int64_t)MAXB * k < ((int64_t)1 << 31) && (int64_t)MAXB * n * 4 < ((int64_t)1 << 31) &&
           2 * w.rb_stride < ((int64_t)1 << 31);
}

MmvParams mmv_params(const WLayout &w, int64_t n, int64_t k) {
    MmvParams p{};
    p.w = w.slab;
    p.wd = w.d;
    p.rb_stride = w.rb_stride;
    p.n = (int)n;
    p.k = (int)k;
    p.ng = w.ng;
    p.nrb = (int)((n + RB - 1) / RB);
    p.tiles = (int)((n + TILE - 1) / TILE);
    p.ks = 1;
    return p;
}

}  // namespace

int mmv_max_k() { return 16384; }

size_t mmv_workspace_bytes(int type, int64_t n, int64_t k) {
    if (type != TYPE_Q4_K || k % QK_K || n <= 0) return 0;
    const Q4kShape q = q4k_shape((int)((n + TILE - 1) / TILE), (int)(k / QK_K));
    return q.ks > 1 ? (size_t)q.ks * MAXB * (size_t)n * 4 : 0;
}

hipError_t launch_mmv(const WLayout &w, int64_t n, int64_t k, const ActPlanes &act, int64_t m, float *y, int32_t *S,
                      int32_t *Smin, void *ws, size_t ws_bytes, hipStream_t s) {
    const int type = w.type;
    if (type != TYPE_Q4_K && type != TYPE_Q6_K) return hipErrorNotSupported;
    if (m < 1 || n <= 0 || k <= 0 || k % QK_K || k > mmv_max_k() || n > 0x7fffffff) return hipErrorNotSupported;
    if (!w.slab || !y || !act.qs || !act.d || !act.bsum16) return hipErrorInvalidValue;
    if (type == TYPE_Q6_K && !w.d) return hipErrorInvalidValue;
    if (w.ng != groups_of(type, k)) return hipErrorInvalidValue;
    if ((S == nullptr) != (Smin == nullptr)) return hipErrorInvalidValue;
    // 32-bit buffer offsets: activation and y of a pass, the tile's two row blocks
    if (!mmv_args_ok(w, n, k)) return hipErrorNotSupported;
    MmvParams p = mmv_params(w, n, k);
    const bool dump = S != nullptr;
    if (type == TYPE_Q4_K) return launch_q4k(p, q4k_shape(p.tiles, p.ng), m, act, y, S, Smin, ws, ws_bytes, s);
    // Q6_K: chunks per tile: about TARGET_WAVES wavefronts in all, chunks of
    // at least MIN_GPC super-blocks, as even as the super-block count allows
    int64_t want = (TARGET_WAVES + p.tiles - 1) / p.tiles;
    want = std::min<int64_t>(want, std::min(MAX_WAVES, std::max(1, p.ng / MIN_GPC)));
    p.gpc = (int)((p.ng + want - 1) / want);
    p.kch = (p.ng + p.gpc - 1) / p.gpc;
    p.tpw = std::max(1, MAX_WAVES / p.kch);  // tiles per workgroup: up to MAX_WAVES wavefronts
    p.iters = (p.tiles + p.tpw - 1) / p.tpw;
    return dump ? launch_f<mmv_kernel<TYPE_Q6_K, true>>(p, p.ng, m, act, y, S, Smin, ws, ws_bytes, s)
                : launch_f<mmv_kernel<TYPE_Q6_K, false>>(p, p.ng, m, act, y, S, Smin, ws, ws_bytes, s);
}

}  // namespace aq
