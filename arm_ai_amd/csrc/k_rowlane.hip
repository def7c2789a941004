// k_rowlane.hip -- batch-1 Q4_K matvec with one weight row per lane, gfx950.
//
// Replaces the column loop of candle-core 0.8.4 k_quants::matmul<BlockQ4K>
// (each output column = BlockQ4K::vec_dot(k, W[col], xq)) for one activation
// row, the decode call at native/arm_ai_nif/src/llama_candle.rs:119, on
// weights with many rows (Llama-3-8B ffn_up / ffn_gate: 14336 x 4096).  The
// integer sums S and Smin of every super-block are exact; only the f32
// combination order differs from candle's vec_dot_unopt.
//
// Mapping.  A workgroup (W = 16 wavefronts) owns 56 consecutive weight rows (seven
// 8-row blocks of the row-block tile layout, so every CU of a 256-CU GPU gets
// the same bytes at the headline shape).  Lane l of every wavefront is row
// row0 + l (lanes 56..63 are idle); wavefront w takes the 256-element groups
// w, w + W, ...  A load instruction therefore reads piece p of one group for
// 56 rows: seven full 128-byte lines.  Because all lanes of a wavefront work
// on the same group, the activation operand of every v_dot4 is the same for
// all lanes: it is read from LDS at a wave-uniform address (one 16-byte
// broadcast read per four v_dot4), so the weights are the only per-lane data.
//
// Schedule.  The first ceil(groups / 4) wavefronts load the activation, then
// every wavefront issues its first P weight pieces, then those wavefronts
// quantise four Q8_K blocks each (16 lanes per block, 16 elements per lane)
// into LDS while the weight pieces are in flight.
// After one barrier each wavefront walks its pieces in order, keeping P of
// them in flight (compute piece j, issue piece j + P): a wavefront never
// waits at the barrier behind its own blocked load issues, and the dot
// products of the pieces that have arrived overlap the rest of the stream.
// Partial sums of a row (one per group) are added across the wavefronts
// through LDS, in wavefront order.
//
// Fewer rows (from 3200; the Llama-3-8B attention projections and ffn_down,
// 4096 rows) with up to 64 groups: a workgroup owns 16 rows and lane l of a
// wavefront is row l % 16 of group phase l / 16, so one load instruction
// reads piece p of four groups for 16 rows (eight full lines) and 256
// workgroups cover 4096 rows.  The activation operand then differs between
// the four 16-lane sets of a wavefront (four broadcast LDS reads), and a
// row's partials are first added across its four lanes, then across the
// wavefronts.
#include "aq_internal.h"

namespace aq {

namespace {

constexpr int RL_ROWS = 56;    // weight rows per workgroup (one row per lane)
constexpr int RL_MAXG = 64;    // groups per row (k <= 16384)
constexpr int RL_MIN_N = 200 * RL_ROWS;  // rows from which 56-row workgroups are used (up to 32 groups)
constexpr int RG_ROWS = 16;    // weight rows per workgroup of the four-group-phase form
constexpr int RG_MIN_N = 200 * RG_ROWS;  // rows from which that form is used (up to 64 groups)

struct RlParams {
    const uint8_t *w;  // row-block tiles
    int64_t rb_stride;
    int n, k, ng;
    const float *x;    // fused: f32 [k]
    ActPlanes act;     // pre-quantised planes (x null)
    float *y;
    int32_t *S, *Smin;  // [n][ng] integer dump, or null
};

template <int CTRL>
__device__ __forceinline__ int dpp_row(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_rowf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// One Q8_K block (candle-core 0.8.4 BlockQ8K::from_float) by the 16 lanes of a
// DPP row: lane s holds elements 16s..16s+15 in v.  Same arithmetic as
// q8k_block_wave (aq_internal.h): max = the first element of largest |x| (NaN
// never wins), iscale = -128/max, q = min(round(iscale*x), 127) ties away
// from zero, d = 1/iscale; an all-zero block gives d = 0, q = 0.  The first
// index of the maximum is found as the smallest key (index << 1 | sign) over
// the row, and its sign gives max = +-amax exactly.  Returns the 16 quants
// packed; *bsum gets the sum of this lane's 16 quants, *d the block's d.
__device__ __forceinline__ uint4 q8k_block_row16(const float v[16], int s, int *bsum, float *d) {
    float ax[16];
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float a = fabsf(v[i]);
        ax[i] = a == a ? a : 0.0f;
        m = fmaxf(m, ax[i]);
    }
    m = fmaxf(m, dpp_rowf<DPP_QUAD_XOR1>(m));
    m = fmaxf(m, dpp_rowf<DPP_QUAD_XOR2>(m));
    m = fmaxf(m, dpp_rowf<DPP_HALF_MIRROR>(m));
    m = fmaxf(m, dpp_rowf<DPP_ROW_MIRROR>(m));
    int q[16];
    float dd = 0.0f;
    if (m != 0.0f) {  // uniform over the row
        int key = 1 << 30;
#pragma unroll
        for (int i = 15; i >= 0; i--)
            if (ax[i] == m) key = ((16 * s + i) << 1) | (v[i] < 0.0f ? 1 : 0);
        key = min(key, dpp_row<DPP_QUAD_XOR1>(key));
        key = min(key, dpp_row<DPP_QUAD_XOR2>(key));
        key = min(key, dpp_row<DPP_HALF_MIRROR>(key));
        key = min(key, dpp_row<DPP_ROW_MIRROR>(key));
        const float mx = (key & 1) ? -m : m;
        const float iscale = -128.0f / mx;
#pragma unroll
        for (int i = 0; i < 16; i++) q[i] = sat_i8(fminf(roundf(iscale * v[i]), 127.0f));
        dd = 1.0f / iscale;
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) q[i] = 0;
    }
    int bs = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) bs += q[i];
    *bsum = bs;
    *d = dd;
    return make_uint4(pack4_i8(q), pack4_i8(q + 4), pack4_i8(q + 8), pack4_i8(q + 12));
}

// R rows per workgroup: RL_ROWS (lane = row, one group phase) or RG_ROWS
// (lane = row + 16 * group phase, four phases).  Lane (row r, phase gp) of
// wavefront w takes the groups w * GP + gp + W * GP * i, i < GPW.
template <int R, int W, int GPW, int P, bool EARLY, bool FUSED, bool DUMP>
__global__ __launch_bounds__(W * 64) void rl_q4k_kernel(RlParams p) {
    static_assert(R == RL_ROWS || R == RG_ROWS, "56 rows, one per lane, or 16 rows in four group phases");
    constexpr int GP = R == RL_ROWS ? 1 : 64 / R;  // group phases per wavefront
    __shared__ __align__(16) uint8_t xq[RL_MAXG][256];  // Q8_K quants of each group
    __shared__ __align__(16) int xb[RL_MAXG][8];        // bsums of the 8 sub-blocks (32 elements)
    __shared__ float xd[RL_MAXG];                       // Q8_K d
    __shared__ float red[W][64];
    constexpr int NP = 9 * GPW;  // this wavefront's pieces, in order
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int rl = GP == 1 ? lane : lane % R, gp = GP == 1 ? 0 : lane / R;
    const int row0 = (int)blockIdx.x * R;
    const int row = row0 + rl;
    const bool rok = rl < R && row < p.n;
    const int rb0 = row0 / RB;
    const int nrb = (p.n + RB - 1) / RB;
    const int rbs = min(R / RB, nrb - rb0);
    const rsrc_t rw = buf_rsrc(p.w + (int64_t)rb0 * p.rb_stride, (uint32_t)(rbs * p.rb_stride));
    const uint32_t lbase = rok ? (uint32_t)((rl / RB) * p.rb_stride + (rl % RB) * 16) : BUF_OOB;
    auto group_of = [&](int j) { return wave * GP + gp + W * GP * (j / 9); };

    uint4 ring[P];
    auto issue = [&](int j) {
        const int g = group_of(j);
        const uint32_t off = g < p.ng ? lbase + (uint32_t)((g * 9 + j % 9) * 128) : BUF_OOB;
        const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, BUF_NT);
        ring[j % P] = make_uint4(t.x, t.y, t.z, t.w);
    };

    // 1. the activation's loads: wavefront w < ceil(ng / 4) stages blocks
    //    4w .. 4w + 3, 16 lanes (s = lane & 15) per block; then (EARLY) this
    //    wavefront's first P weight pieces, so that they are in flight while
    //    the activation is quantised (the loads are waited for in issue
    //    order).  With most wavefronts quantising (the 16-wavefront form),
    //    issuing them after the quantisation measured faster.
    const int s = lane & 15;
    const int gb = 4 * wave + (lane >> 4);
    const bool quantiser = wave < (p.ng + 3) / 4;  // uniform
    const bool gbok = gb < p.ng;
    u32x4 xv[4];
    uint32_t xbs = 0, xdb = 0;
    if (quantiser) {
        if (FUSED) {
            const rsrc_t rx = buf_rsrc(p.x, (uint32_t)(p.k * 4));
            const uint32_t xo = gbok ? (uint32_t)((gb * QK_K + 16 * s) * 4) : BUF_OOB;
#pragma unroll
            for (int i = 0; i < 4; i++) xv[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 16 * i, 0, 0);
        } else {
            const rsrc_t rq = buf_rsrc(p.act.qs, (uint32_t)p.k);
            const rsrc_t rs = buf_rsrc(p.act.bsums, (uint32_t)((p.k / 16) * 2));
            const rsrc_t rd = buf_rsrc(p.act.d, (uint32_t)((p.k / QK_K) * 4));
            xv[0] = __builtin_amdgcn_raw_buffer_load_b128(rq, gbok ? (uint32_t)(gb * QK_K + 16 * s) : BUF_OOB, 0, 0);
            xbs = __builtin_amdgcn_raw_buffer_load_b16(rs, gbok ? (uint32_t)((gb * 16 + s) * 2) : BUF_OOB, 0, 0);
            xdb = __builtin_amdgcn_raw_buffer_load_b32(rd, gbok ? (uint32_t)(gb * 4) : BUF_OOB, 0, 0);
        }
    }
    if (EARLY) {
#pragma unroll
        for (int j = 0; j < P && j < NP; j++) issue(j);
    }
    // 2. quantise (or unpack) into LDS, then one barrier (LDS writes only)
    if (quantiser) {
        uint4 qv;
        int bsum;
        float d;
        if (FUSED) {
            float v[16];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[4 * i] = u32_as_f32(xv[i].x);
                v[4 * i + 1] = u32_as_f32(xv[i].y);
                v[4 * i + 2] = u32_as_f32(xv[i].z);
                v[4 * i + 3] = u32_as_f32(xv[i].w);
            }
            qv = q8k_block_row16(v, s, &bsum, &d);
        } else {
            qv = make_uint4(xv[0].x, xv[0].y, xv[0].z, xv[0].w);
            bsum = (int)(int16_t)xbs;
            d = u32_as_f32(xdb);
        }
        const int pair = bsum + dpp_row<DPP_QUAD_XOR1>(bsum);  // sub-block s/2 (two 16-element halves)
        if (gbok) {
            *(uint4 *)&xq[gb][16 * s] = qv;
            if ((s & 1) == 0) xb[gb][s >> 1] = pair;
            if (s == 0) xd[gb] = d;
        }
    }
    if (!EARLY) {
#pragma unroll
        for (int j = 0; j < P && j < NP; j++) issue(j);
    }
    lds_barrier();

    // 3. walk the pieces: piece 0 of a group = d, dmin, 12 scale bytes; piece
    //    1 + 2c + h = qs bytes 32c + 16h .. +15 (low nibbles: elements
    //    64c + 16h + i of sub-block 2c; high: 64c + 32 + 16h + i of 2c + 1)
    float f = 0.0f;
    int bs[8];
    float dx = 0.0f;
    uint32_t sc03 = 0, sc47 = 0, mn03 = 0, mn47 = 0, dwp = 0;
    int S = 0, il = 0, ih = 0;
#pragma unroll
    for (int j = 0; j < NP; j++) {
        const int pc = j % 9;
        const int g = group_of(j);
        if (GP == 1 && g >= p.ng) break;  // uniform
        const bool gok = g < p.ng;         // (lanes of several phases: per lane)
        const int gl = gok ? g : 0;        // a group whose LDS entries are written
        const uint4 q = ring[j % P];
        if (pc == 0) {
            *(int4 *)&bs[0] = *(const int4 *)&xb[gl][0];
            *(int4 *)&bs[4] = *(const int4 *)&xb[gl][4];
            dx = xd[gl];
            // candle's utmp form of GGML get_scale_min_k4 (6-bit scales and mins)
            const uint32_t u0 = q.y, u1 = q.z, u2 = q.w;
            sc03 = u0 & 0x3F3F3F3Fu;
            sc47 = (u2 & 0x0F0F0F0Fu) | (((u0 >> 6) & 0x03030303u) << 4);
            mn03 = u1 & 0x3F3F3F3Fu;
            mn47 = ((u2 >> 4) & 0x0F0F0F0Fu) | (((u1 >> 6) & 0x03030303u) << 4);
            dwp = q.x;
            S = 0;
        } else {
            const int c = (pc - 1) >> 1, h = (pc - 1) & 1;
            // x of the low nibbles (elements 64c + 16h ..) and of the high
            // nibbles (64c + 32 + 16h ..): the same for every lane
            const int4 xl = *(const int4 *)&xq[gl][64 * c + 16 * h];
            const int4 xh = *(const int4 *)&xq[gl][64 * c + 32 + 16 * h];
            if (h == 0) il = ih = 0;
            il = sdot4((int)(q.x & 0x0F0F0F0Fu), xl.x, il);
            ih = sdot4((int)((q.x >> 4) & 0x0F0F0F0Fu), xh.x, ih);
            il = sdot4((int)(q.y & 0x0F0F0F0Fu), xl.y, il);
            ih = sdot4((int)((q.y >> 4) & 0x0F0F0F0Fu), xh.y, ih);
            il = sdot4((int)(q.z & 0x0F0F0F0Fu), xl.z, il);
            ih = sdot4((int)((q.z >> 4) & 0x0F0F0F0Fu), xh.z, ih);
            il = sdot4((int)(q.w & 0x0F0F0F0Fu), xl.w, il);
            ih = sdot4((int)((q.w >> 4) & 0x0F0F0F0Fu), xh.w, ih);
            if (h == 1) {
                const uint32_t sw = c < 2 ? sc03 : sc47;
                S += (int)((sw >> (16 * (c & 1))) & 0xffu) * il + (int)((sw >> (16 * (c & 1) + 8)) & 0xffu) * ih;
            }
        }
        if (j + P < NP) issue(j + P);
        if (pc == 8) {
            int smin = 0;
#pragma unroll
            for (int jj = 0; jj < 8; jj++) smin += (int)(((jj < 4 ? mn03 : mn47) >> (8 * (jj & 3))) & 0xffu) * bs[jj];
            const float dw = f16_bits_to_f32(dwp), dmw = f16_bits_to_f32(dwp >> 16);
            if (gok) f += (dw * dx) * (float)S - (dmw * dx) * (float)smin;
            if (DUMP && rok && gok) {
                p.S[(int64_t)row * p.ng + g] = S;
                p.Smin[(int64_t)row * p.ng + g] = smin;
            }
        }
    }
    // 4. the row's partials: over its group phases within the wavefront,
    //    then over the wavefronts, in wavefront order
    if (GP == 4) f += __shfl_xor(f, 16);
    if (GP >= 2) f += __shfl_xor(f, 32);
    red[wave][lane] = f;
    lds_barrier();
    if (wave == 0 && rok && gp == 0) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) t += red[w][lane];
        p.y[row] = t;
    }
}

template <int R, int W, int GPW, int P, bool EARLY>
hipError_t launch_g(const RlParams &p, unsigned grid, bool fused, bool dump, hipStream_t s) {
    if (fused) {
        if (dump) rl_q4k_kernel<R, W, GPW, P, EARLY, true, true><<<grid, W * 64, 0, s>>>(p);
        else rl_q4k_kernel<R, W, GPW, P, EARLY, true, false><<<grid, W * 64, 0, s>>>(p);
    } else {
        if (dump) rl_q4k_kernel<R, W, GPW, P, EARLY, false, true><<<grid, W * 64, 0, s>>>(p);
        else rl_q4k_kernel<R, W, GPW, P, EARLY, false, false><<<grid, W * 64, 0, s>>>(p);
    }
    return hipGetLastError();
}

bool rows56(int64_t n, int ng) { return ng <= 32 && n >= RL_MIN_N; }

}  // namespace

bool rowlane_matvec_applies(int type, int64_t n, int64_t k) {
    return type == TYPE_Q4_K && k % QK_K == 0 && k > 0 && k / QK_K <= RL_MAXG && n <= 0x7fffffff &&
           (rows56(n, (int)(k / QK_K)) || n >= RG_MIN_N);
}

hipError_t launch_rowlane_matvec(const WLayout &w, int64_t n, int64_t k, const float *x, const ActPlanes *act,
                                 float *y, int32_t *S, int32_t *Smin, hipStream_t s) {
    if (!rowlane_matvec_applies(w.type, n, k)) return hipErrorNotSupported;
    if (!w.slab || !y || (!x && !act) || (S == nullptr) != (Smin == nullptr)) return hipErrorInvalidValue;
    const int ng = (int)(k / QK_K);
    if (w.ng != ng || w.rb_stride != (int64_t)ng * 9 * 128) return hipErrorInvalidValue;
    if (x && ((uintptr_t)x & 15)) return hipErrorInvalidValue;
    const bool wide = rows56(n, ng);
    if ((int64_t)(wide ? RL_ROWS : RG_ROWS) / RB * w.rb_stride >= ((int64_t)1 << 31)) return hipErrorNotSupported;
    RlParams p;
    p.w = w.slab;
    p.rb_stride = w.rb_stride;
    p.n = (int)n;
    p.k = (int)k;
    p.ng = ng;
    p.x = x;
    p.act = act ? *act : ActPlanes{};
    p.y = y;
    p.S = S;
    p.Smin = Smin;
    const bool fused = x != nullptr, dump = S != nullptr;
    if (wide) {
        const unsigned grid = (unsigned)((n + RL_ROWS - 1) / RL_ROWS);
        // 16 wavefronts with six pieces in flight each measured fastest at the
        // headline (one group per wavefront); longer rows take two groups each
        if (ng <= 16) return launch_g<RL_ROWS, 16, 1, 6, true>(p, grid, fused, dump, s);
        return launch_g<RL_ROWS, 16, 2, 12, true>(p, grid, fused, dump, s);
    }
    // 16 rows: as many wavefronts as four groups each need (every lane one
    // group); the quantising wavefronts (four blocks each) are then always
    // enough.  Up to 32 groups all nine pieces of a lane's group are in
    // flight from the start; with 16 wavefronts (ffn_down, 56 groups) five,
    // issued after the quantisation, measured fastest (8.3 us against 8.6
    // for nine issued late and 9.7 for nine issued early).
    const unsigned grid = (unsigned)((n + RG_ROWS - 1) / RG_ROWS);
    if (ng <= 16) return launch_g<RG_ROWS, 4, 1, 9, true>(p, grid, fused, dump, s);
    if (ng <= 32) return launch_g<RG_ROWS, 8, 1, 9, true>(p, grid, fused, dump, s);
    return launch_g<RG_ROWS, 16, 1, 5, false>(p, grid, fused, dump, s);
}

}  // namespace aq
