// k_matvec.hip -- decode-path matvec (batch 1..8 per pass) for Q4_K / Q6_K /
// Q8_0 weights against Q8_K / Q8_0 activations, gfx950.
//
// Replaces the column loop of candle-core 0.8.4 k_quants::matmul<T> (each
// output column = T::vec_dot(k, W[col], xq[row])), reached from
// native/arm_ai_nif/src/llama_candle.rs:119 at decode.  The integer part of
// every block dot product is computed exactly (v_dot4_i32_i8 on 4 bytes at a
// time); only the f32 combination order differs from candle's vec_dot_unopt.
//
// Mapping.  One lane owns one 256-element group (a Q4_K/Q6_K super-block, or
// eight Q8_0 blocks) of one weight row per iteration.  The lanes of a "row
// group" (lpr = next power of two >= groups per row, at most 64) cover a
// whole row, so a wavefront covers 64/lpr rows, and the loads of piece i of
// all its groups are one contiguous slab read (the weight layout is described
// in aq_internal.h).  Each wavefront prefetches the weights of its next
// iteration before computing the current one.  The activation (all batch rows
// of the pass) sits in LDS as one 304-byte record per (row, group); the
// records' stride spreads the 16-byte reads of consecutive lanes over
// disjoint LDS banks.  With an f32 input the workgroup quantises it into LDS
// itself (same device code as the quantizer kernels, so the same bytes)
// while its first weight loads are in flight.
#include "aq_internal.h"

namespace aq {

namespace {

constexpr int REC = 304;           // LDS bytes per (batch row, group) activation record
constexpr int REC_BSUMS = 256;     // Q8_K record: i16 bsums[16]
constexpr int REC_D = 288;         // Q8_K record: f32 d
constexpr int REC_D8 = 256;        // Q8_0 record: f32 d[8] (value of the f16 d)
constexpr size_t LDS_CAP = 64 * 1024;
constexpr int TARGET_WAVES = 4096;  // about 16 wavefronts per CU on 256 CUs

struct MvParams {
    const uint8_t *w;    // slab plane
    const uint16_t *wd;  // Q6_K d plane
    int64_t row_bytes;
    int n, k, ng, lpr_log, m, iters, nwaves;
    const float *x;      // fused: f32 [m][k] of this pass, or null
    ActPlanes act;       // pre-quantised planes of this pass (when x is null)
    float *y;            // [m][n] of this pass
    int32_t *S, *Smin;   // [m][n][blocks] of this pass, or null
};

template <int TYPE>
struct Wt {
    uint4 pc[slabs_of(TYPE)];
    uint32_t d;  // Q6_K super-block d (f16 bits)
};

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Weights are streamed once per call: nontemporal loads keep them from
// displacing the (reused) activation in the caches.
template <int TYPE>
__device__ __forceinline__ void load_w(Wt<TYPE> &W, const MvParams &p, int row, int g) {
    const uint8_t *base = p.w + (int64_t)row * p.row_bytes + (int64_t)g * 16;
    const int64_t stride = (int64_t)p.ng * 16;
#pragma unroll
    for (int i = 0; i < slabs_of(TYPE); i++) {
        const u32x4 t = __builtin_nontemporal_load((const u32x4 *)(base + i * stride));
        W.pc[i] = make_uint4(t.x, t.y, t.z, t.w);
    }
    if (TYPE == TYPE_Q6_K) W.d = p.wd[(int64_t)row * p.ng + g];
}

template <int TYPE>
__device__ __forceinline__ void zero_w(Wt<TYPE> &W) {
#pragma unroll
    for (int i = 0; i < slabs_of(TYPE); i++) W.pc[i] = make_uint4(0, 0, 0, 0);
    W.d = 0;
}

__device__ __forceinline__ int byte_u(uint32_t w, int i) { return (int)((w >> (8 * i)) & 0xffu); }
__device__ __forceinline__ int byte_s(uint32_t w, int i) { return (int)(int8_t)(w >> (8 * i)); }
__device__ __forceinline__ int lo16(uint32_t w) { return (int)(int16_t)(w & 0xffffu); }
__device__ __forceinline__ int hi16(uint32_t w) { return (int)(int16_t)(w >> 16); }

__device__ __forceinline__ int dot16(const uint32_t q[4], const int4 x, int acc) {
    acc = sdot4((int)q[0], x.x, acc);
    acc = sdot4((int)q[1], x.y, acc);
    acc = sdot4((int)q[2], x.z, acc);
    acc = sdot4((int)q[3], x.w, acc);
    return acc;
}

// ------------------------------------------------------------------ Q4_K
// Super-block: piece 0 = d, dmin, 12 scale bytes; piece 1 + 2c + h = qs bytes
// 32c + 16h .. +15, whose low nibbles are elements 64c + 16h + i (sub-block
// 2c) and high nibbles elements 64c + 32 + 16h + i (sub-block 2c + 1).
template <int B, bool DUMP>
__device__ __forceinline__ void dot_q4k(const Wt<TYPE_Q4_K> &W, const uint8_t *lds, int ng, int g, int m,
                                        float (&f)[B], int (&So)[B], int (&Smo)[B]) {
    const uint32_t u0 = W.pc[0].y, u1 = W.pc[0].z, u2 = W.pc[0].w;
    // candle's utmp form of GGML get_scale_min_k4 (6-bit scales and mins)
    const uint32_t sc03 = u0 & 0x3F3F3F3Fu;
    const uint32_t sc47 = (u2 & 0x0F0F0F0Fu) | (((u0 >> 6) & 0x03030303u) << 4);
    const uint32_t mn03 = u1 & 0x3F3F3F3Fu;
    const uint32_t mn47 = ((u2 >> 4) & 0x0F0F0F0Fu) | (((u1 >> 6) & 0x03030303u) << 4);
    const float dw = f16_bits_to_f32(W.pc[0].x), dmw = f16_bits_to_f32(W.pc[0].x >> 16);
    int S[B];
#pragma unroll
    for (int b = 0; b < B; b++) S[b] = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        int il[B], ih[B];
#pragma unroll
        for (int b = 0; b < B; b++) il[b] = ih[b] = 0;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint4 q = W.pc[1 + 2 * c + h];
            const uint32_t lo[4] = {q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu, q.z & 0x0F0F0F0Fu, q.w & 0x0F0F0F0Fu};
            const uint32_t hi[4] = {(q.x >> 4) & 0x0F0F0F0Fu, (q.y >> 4) & 0x0F0F0F0Fu, (q.z >> 4) & 0x0F0F0F0Fu,
                                    (q.w >> 4) & 0x0F0F0F0Fu};
#pragma unroll
            for (int b = 0; b < B; b++) {
                if (b < m) {
                    const uint8_t *rec = lds + (b * ng + g) * REC + 64 * c + 16 * h;
                    il[b] = dot16(lo, *(const int4 *)rec, il[b]);
                    ih[b] = dot16(hi, *(const int4 *)(rec + 32), ih[b]);
                }
            }
        }
        const uint32_t sw = c < 2 ? sc03 : sc47;
        const int s_lo = byte_u(sw, 2 * (c & 1)), s_hi = byte_u(sw, 2 * (c & 1) + 1);
#pragma unroll
        for (int b = 0; b < B; b++) S[b] += s_lo * il[b] + s_hi * ih[b];
    }
#pragma unroll
    for (int b = 0; b < B; b++) {
        if (b < m) {
            const uint8_t *rec = lds + (b * ng + g) * REC;
            const int4 p0 = *(const int4 *)(rec + REC_BSUMS), p1 = *(const int4 *)(rec + REC_BSUMS + 16);
            // bsums dword j holds bsums[2j], bsums[2j+1]: the two halves of sub-block j
            const uint32_t pw[8] = {(uint32_t)p0.x, (uint32_t)p0.y, (uint32_t)p0.z, (uint32_t)p0.w,
                                    (uint32_t)p1.x, (uint32_t)p1.y, (uint32_t)p1.z, (uint32_t)p1.w};
            int smin = 0;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int mj = byte_u(j < 4 ? mn03 : mn47, j & 3);
                smin += mj * (lo16(pw[j]) + hi16(pw[j]));
            }
            const float dx = *(const float *)(rec + REC_D);
            f[b] += (dw * dx) * (float)S[b] - (dmw * dx) * (float)smin;
            if (DUMP) {
                So[b] = S[b];
                Smo[b] = smin;
            }
        }
    }
}

// ------------------------------------------------------------------ Q6_K
// Super-block: pieces 0..7 = ql, 8..11 = qh, 12 = the 16 int8 sub-scales.
// For half hh and 16-element half t, pieces A = ql[4hh + t], Bq = ql[4hh + 2 + t]
// and H = qh[2hh + t] hold elements 128hh + 32gq + 16t + i (gq = 0..3):
//   gq0: A & 0xF | (H & 3) << 4        gq1: Bq & 0xF | (H >> 2 & 3) << 4
//   gq2: A >> 4 | (H >> 4 & 3) << 4    gq3: Bq >> 4 | (H >> 6 & 3) << 4
// each minus 32; sub-block of element e is e/16 = 8hh + 2gq + t.
template <int B, bool DUMP>
__device__ __forceinline__ void dot_q6k(const Wt<TYPE_Q6_K> &W, const uint8_t *lds, int ng, int g, int m,
                                        float (&f)[B], int (&So)[B], int (&Smo)[B]) {
    const uint32_t scw[4] = {W.pc[12].x, W.pc[12].y, W.pc[12].z, W.pc[12].w};
    int S[B];
#pragma unroll
    for (int b = 0; b < B; b++) S[b] = 0;
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const uint4 A = W.pc[4 * hh + t], Bq = W.pc[4 * hh + 2 + t], H = W.pc[8 + 2 * hh + t];
            const uint32_t a[4] = {A.x, A.y, A.z, A.w}, bq[4] = {Bq.x, Bq.y, Bq.z, Bq.w}, hq[4] = {H.x, H.y, H.z, H.w};
            uint32_t q[4][4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                q[0][i] = (a[i] & 0x0F0F0F0Fu) | ((hq[i] << 4) & 0x30303030u);
                q[1][i] = (bq[i] & 0x0F0F0F0Fu) | ((hq[i] << 2) & 0x30303030u);
                q[2][i] = ((a[i] >> 4) & 0x0F0F0F0Fu) | (hq[i] & 0x30303030u);
                q[3][i] = ((bq[i] >> 4) & 0x0F0F0F0Fu) | ((hq[i] >> 2) & 0x30303030u);
            }
#pragma unroll
            for (int b = 0; b < B; b++) {
                if (b < m) {
                    const uint8_t *rec = lds + (b * ng + g) * REC;
#pragma unroll
                    for (int gq = 0; gq < 4; gq++) {
                        const int j = 8 * hh + 2 * gq + t;
                        const int isum = dot16(q[gq], *(const int4 *)(rec + 16 * j), 0);
                        const int bs = (int)*(const int16_t *)(rec + REC_BSUMS + 2 * j);
                        // sum (q6 - 32) * x = sum q6 * x - 32 * (sum of the same 16 x)
                        S[b] += byte_s(scw[j >> 2], j & 3) * (isum - 32 * bs);
                    }
                }
            }
        }
    }
    const float dw = f16_bits_to_f32(W.d);
#pragma unroll
    for (int b = 0; b < B; b++) {
        if (b < m) {
            const float dx = *(const float *)(lds + (b * ng + g) * REC + REC_D);
            f[b] += (dw * dx) * (float)S[b];
            if (DUMP) {
                So[b] = S[b];
                Smo[b] = 0;
            }
        }
    }
}

// ------------------------------------------------------------------ Q8_0
// Group of eight blocks: pieces 2j, 2j+1 = qs of block j, piece 16 = the
// eight f16 d.  candle: sumf += (sum_i qw*qx as f32) * f16(d_w) * f16(d_x).
template <int B, bool DUMP>
__device__ __forceinline__ void dot_q80(const Wt<TYPE_Q8_0> &W, const uint8_t *lds, int ng, int g, int m,
                                        float (&f)[B], const MvParams &p, int row) {
    const uint32_t dwp[4] = {W.pc[16].x, W.pc[16].y, W.pc[16].z, W.pc[16].w};
    const int nblk = p.k / QK8_0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint4 q0 = W.pc[2 * j], q1 = W.pc[2 * j + 1];
        const uint32_t qa[4] = {q0.x, q0.y, q0.z, q0.w}, qb[4] = {q1.x, q1.y, q1.z, q1.w};
        const float dw = f16_bits_to_f32(dwp[j >> 1] >> (16 * (j & 1)));
#pragma unroll
        for (int b = 0; b < B; b++) {
            if (b < m) {
                const uint8_t *rec = lds + (b * ng + g) * REC;
                int isum = dot16(qa, *(const int4 *)(rec + 32 * j), 0);
                isum = dot16(qb, *(const int4 *)(rec + 32 * j + 16), isum);
                const float dx = *(const float *)(rec + REC_D8 + 4 * j);
                f[b] += ((float)isum * dw) * dx;
                if (DUMP) {
                    const int blk = 8 * g + j;
                    if (blk < nblk) {
                        const int64_t o = ((int64_t)b * p.n + row) * nblk + blk;
                        p.S[o] = isum;
                        p.Smin[o] = 0;
                    }
                }
            }
        }
    }
}

template <int TYPE, int B, bool DUMP>
__device__ __forceinline__ void group_dot(const Wt<TYPE> &W, const uint8_t *lds, const MvParams &p, int g, int row,
                                          bool valid, float (&f)[B]) {
    if (TYPE == TYPE_Q8_0) {
        dot_q80<B, DUMP && true>(*(const Wt<TYPE_Q8_0> *)&W, lds, p.ng, g, p.m, f, p, row);
        (void)valid;
    } else {
        int So[B], Smo[B];
        if (TYPE == TYPE_Q4_K) dot_q4k<B, DUMP>(*(const Wt<TYPE_Q4_K> *)&W, lds, p.ng, g, p.m, f, So, Smo);
        else dot_q6k<B, DUMP>(*(const Wt<TYPE_Q6_K> *)&W, lds, p.ng, g, p.m, f, So, Smo);
        if (DUMP && valid) {
#pragma unroll
            for (int b = 0; b < B; b++) {
                if (b < p.m) {
                    const int64_t o = ((int64_t)b * p.n + row) * p.ng + g;
                    p.S[o] = So[b];
                    p.Smin[o] = Smo[b];
                }
            }
        }
    }
}

// Activation of this pass into LDS records.  The global loads of the first
// PRE records of each wave (rec_load) are issued before the weight loads of
// the first iteration, so quantising them (rec_store) waits only for them.
constexpr int NW = 8;    // wavefronts per workgroup
constexpr int PRE = 4;   // records per wave whose loads precede the weight loads

struct ActStage {
    float4 v[PRE];
    int4 q[PRE];
    float dsc[PRE];
};

template <int TYPE>
__device__ __forceinline__ void rec_load(ActStage &st, int r, const MvParams &p, int t, int lane) {
    const int ng = p.ng, k = p.k;
    const int b = t / ng, g = t - b * ng;
    if (p.x) {
        if (TYPE != TYPE_Q8_0) {
            st.v[r] = *(const float4 *)(p.x + (int64_t)b * k + g * QK_K + 4 * lane);
        } else {
            const int j = lane >> 3, sub = lane & 7;
            st.v[r] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if ((8 * g + j) * QK8_0 < k) st.v[r] = *(const float4 *)(p.x + (int64_t)b * k + (8 * g + j) * QK8_0 + 4 * sub);
        }
    } else {
        st.q[r] = make_int4(0, 0, 0, 0);
        st.dsc[r] = 0.0f;
        if (TYPE != TYPE_Q8_0) {
            if (lane < 16) st.q[r] = *(const int4 *)(p.act.qs + (int64_t)b * k + g * QK_K + 16 * lane);
            else if (lane < 18) st.q[r] = *(const int4 *)(p.act.bsums + (int64_t)b * (k / 16) + g * 16 + 8 * (lane - 16));
            else if (lane == 18) st.dsc[r] = p.act.d[(int64_t)b * (k / QK_K) + g];
        } else {
            const int nblk = k / QK8_0;
            if (lane < 16) {
                const int j = lane >> 1;
                if (8 * g + j < nblk) st.q[r] = *(const int4 *)(p.act.qs + (int64_t)b * k + (8 * g + j) * QK8_0 + 16 * (lane & 1));
            } else if (lane < 24) {
                const int j = lane - 16;
                if (8 * g + j < nblk) st.dsc[r] = p.act.d[(int64_t)b * nblk + 8 * g + j];
            }
        }
    }
}

template <int TYPE>
__device__ __forceinline__ void rec_store(const ActStage &st, int r, uint8_t *lds, const MvParams &p, int t, int lane) {
    uint8_t *rec = lds + t * REC;
    if (p.x) {
        const float v[4] = {st.v[r].x, st.v[r].y, st.v[r].z, st.v[r].w};
        if (TYPE != TYPE_Q8_0) {
            int bsum;
            float d;
            const uint32_t packed = q8k_block_wave(v, lane, &bsum, &d);
            *(uint32_t *)(rec + 4 * lane) = packed;
            if ((lane & 3) == 0) *(int16_t *)(rec + REC_BSUMS + 2 * (lane >> 2)) = (int16_t)bsum;
            if (lane == 0) *(float *)(rec + REC_D) = d;
        } else {
            const int j = lane >> 3, sub = lane & 7;
            uint16_t h;
            const uint32_t packed = q8_0_block_8lanes(v, &h);  // a padding block is all zeros: q = 0, d = 0
            *(uint32_t *)(rec + 32 * j + 4 * sub) = packed;
            if (sub == 0) *(float *)(rec + REC_D8 + 4 * j) = f16_bits_to_f32(h);
        }
    } else {
        if (TYPE != TYPE_Q8_0) {
            if (lane < 16) *(int4 *)(rec + 16 * lane) = st.q[r];
            else if (lane < 18) *(int4 *)(rec + REC_BSUMS + 16 * (lane - 16)) = st.q[r];
            else if (lane == 18) *(float *)(rec + REC_D) = st.dsc[r];
        } else {
            if (lane < 16) *(int4 *)(rec + 16 * lane) = st.q[r];
            else if (lane < 24) *(float *)(rec + REC_D8 + 4 * (lane - 16)) = st.dsc[r];
        }
    }
}

template <int TYPE, int B, bool DUMP, bool MULTI>
__global__ __launch_bounds__(NW * 64) void matvec_kernel(MvParams p) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lpr = 1 << p.lpr_log, rpw = 64 >> p.lpr_log;
    const int sl = lane & (lpr - 1), grp = lane >> p.lpr_log;
    const int gw = blockIdx.x * NW + wave;
    const int iters = gw < p.nwaves ? p.iters : 0;
    const int nrec = p.m * p.ng;

    // 1. activation loads of the first records, 2. weight loads of the first
    // iteration, 3. quantise / copy into LDS (waits only for step 1).
    ActStage st;
#pragma unroll
    for (int r = 0; r < PRE; r++) {
        const int t = wave + NW * r;
        if (t < nrec) rec_load<TYPE>(st, r, p, t, lane);
    }
    Wt<TYPE> wa, wb;
    int row = gw * rpw + grp;
    bool valid = iters > 0 && row < p.n && sl < p.ng;
    if (!MULTI) {
        if (valid) load_w<TYPE>(wa, p, row, sl);
        else zero_w<TYPE>(wa);
    }
#pragma unroll
    for (int r = 0; r < PRE; r++) {
        const int t = wave + NW * r;
        if (t < nrec) rec_store<TYPE>(st, r, lds, p, t, lane);
    }
    for (int t = wave + NW * PRE; t < nrec; t += NW) {
        rec_load<TYPE>(st, 0, p, t, lane);
        rec_store<TYPE>(st, 0, lds, p, t, lane);
    }
    __syncthreads();

    auto finish = [&](float (&f)[B], int r) {
        // reduce over the lanes of the row group (aligned groups of lpr lanes)
#pragma unroll
        for (int b = 0; b < B; b++)
            for (int off = lpr >> 1; off >= 1; off >>= 1) f[b] += __shfl_xor(f[b], off);
        if (sl == 0 && r < p.n) {
#pragma unroll
            for (int b = 0; b < B; b++)
                if (b < p.m) p.y[(int64_t)b * p.n + r] = f[b];
        }
    };

    if (!MULTI) {
        // ping-pong: wa holds iteration it, wb iteration it + 1
        for (int it = 0; it < iters; it += 2) {
            const int row_b = (gw + (it + 1) * p.nwaves) * rpw + grp;
            const bool valid_b = it + 1 < iters && row_b < p.n && sl < p.ng;
            if (valid_b) load_w<TYPE>(wb, p, row_b, sl);
            float f[B];
#pragma unroll
            for (int b = 0; b < B; b++) f[b] = 0.0f;
            if (valid) group_dot<TYPE, B, DUMP>(wa, lds, p, sl, row, true, f);
            finish(f, row);
            if (it + 1 >= iters) break;
            row = (gw + (it + 2) * p.nwaves) * rpw + grp;
            valid = it + 2 < iters && row < p.n && sl < p.ng;
            if (valid) load_w<TYPE>(wa, p, row, sl);
#pragma unroll
            for (int b = 0; b < B; b++) f[b] = 0.0f;
            if (valid_b) group_dot<TYPE, B, DUMP>(wb, lds, p, sl, row_b, true, f);
            finish(f, row_b);
        }
    } else {
        for (int it = 0; it < iters; it++) {
            float f[B];
#pragma unroll
            for (int b = 0; b < B; b++) f[b] = 0.0f;
            if (row < p.n) {
                for (int g = sl; g < p.ng; g += 64) {
                    load_w<TYPE>(wb, p, row, g);
                    group_dot<TYPE, B, DUMP>(wb, lds, p, g, row, true, f);
                }
            }
            finish(f, row);
            row = (gw + (it + 1) * p.nwaves) * rpw + grp;
        }
    }
}

template <int TYPE, int B>
hipError_t launch_tb(const MvParams &p, unsigned grid, size_t lds, bool dump, bool multi, hipStream_t s) {
    if (dump) {
        if (multi) matvec_kernel<TYPE, B, true, true><<<grid, NW * 64, lds, s>>>(p);
        else matvec_kernel<TYPE, B, true, false><<<grid, NW * 64, lds, s>>>(p);
    } else {
        if (multi) matvec_kernel<TYPE, B, false, true><<<grid, NW * 64, lds, s>>>(p);
        else matvec_kernel<TYPE, B, false, false><<<grid, NW * 64, lds, s>>>(p);
    }
    return hipGetLastError();
}

template <int TYPE>
hipError_t launch_t(int B, const MvParams &p, unsigned grid, size_t lds, bool dump, bool multi, hipStream_t s) {
    switch (B) {
    case 1: return launch_tb<TYPE, 1>(p, grid, lds, dump, multi, s);
    case 2: return launch_tb<TYPE, 2>(p, grid, lds, dump, multi, s);
    case 4: return launch_tb<TYPE, 4>(p, grid, lds, dump, multi, s);
    case 8: return launch_tb<TYPE, 8>(p, grid, lds, dump, multi, s);
    default: return hipErrorInvalidConfiguration;
    }
}

}  // namespace

hipError_t launch_matvec(const WLayout &w, int64_t n, int64_t k, const float *x, const ActPlanes *act, int64_t m,
                         float *y, int32_t *S, int32_t *Smin, hipStream_t s) {
    const int type = w.type;
    if (type != TYPE_Q4_K && type != TYPE_Q6_K && type != TYPE_Q8_0) return hipErrorInvalidValue;
    const int blk = type == TYPE_Q8_0 ? QK8_0 : QK_K;
    if (!w.slab || m < 0 || n <= 0 || k <= 0 || k % blk || n > 0x7fffffff || k > 0x7fffffff || !y)
        return hipErrorInvalidValue;
    if (type == TYPE_Q6_K && !w.d) return hipErrorInvalidValue;
    if (w.ng != groups_of(type, k)) return hipErrorInvalidValue;
    if (!x && !act) return hipErrorInvalidValue;
    if (x && ((uintptr_t)x & 15)) return hipErrorInvalidValue;  // the fused prologue reads float4
    if ((S == nullptr) != (Smin == nullptr)) return hipErrorInvalidValue;
    if (m == 0) return hipSuccess;
    const int ng = w.ng;
    if ((size_t)ng * REC > LDS_CAP) return hipErrorNotSupported;  // k > 55040
    int lpr_log = 0;
    while ((1 << lpr_log) < ng && lpr_log < 6) lpr_log++;
    const bool multi = ng > 64;
    const int rpw = 64 >> lpr_log;
    const int64_t ri = (n + rpw - 1) / rpw;  // wavefront iterations
    const int64_t iters = (ri + TARGET_WAVES - 1) / TARGET_WAVES;
    const int64_t nwaves = (ri + iters - 1) / iters;
    const int64_t grid = (nwaves + NW - 1) / NW;
    const int64_t nblk = k / blk;
    int64_t r0 = 0;
    while (r0 < m) {
        const int64_t rem = m - r0;
        int B = rem >= 8 ? 8 : rem > 4 ? 8 : rem > 2 ? 4 : rem;
        while (B > 1 && (size_t)B * ng * REC > LDS_CAP) B >>= 1;
        const int mb = (int)(rem < B ? rem : B);
        MvParams p;
        p.w = w.slab;
        p.wd = w.d;
        p.row_bytes = w.row_bytes;
        p.n = (int)n;
        p.k = (int)k;
        p.ng = ng;
        p.lpr_log = lpr_log;
        p.m = mb;
        p.iters = (int)iters;
        p.nwaves = (int)nwaves;
        p.x = x ? x + r0 * k : nullptr;
        if (act) {
            p.act.qs = act->qs + r0 * k;
            p.act.d = act->d + r0 * (k / blk);
            p.act.d16 = act->d16;
            p.act.bsums = act->bsums + r0 * (k / 16);
        } else {
            p.act = ActPlanes{};
        }
        p.y = y + r0 * n;
        p.S = S ? S + r0 * n * nblk : nullptr;
        p.Smin = Smin ? Smin + r0 * n * nblk : nullptr;
        const size_t lds = (size_t)B * ng * REC;
        hipError_t e;
        switch (type) {
        case TYPE_Q4_K: e = launch_t<TYPE_Q4_K>(B, p, (unsigned)grid, lds, S != nullptr, multi, s); break;
        case TYPE_Q6_K: e = launch_t<TYPE_Q6_K>(B, p, (unsigned)grid, lds, S != nullptr, multi, s); break;
        default: e = launch_t<TYPE_Q8_0>(B, p, (unsigned)grid, lds, S != nullptr, multi, s); break;
        }
        if (e != hipSuccess) return e;
        r0 += mb;
    }
    return hipSuccess;
}

}  // namespace aq
