// k_rowlane.hip -- batch-1 matvec with one weight row per lane, gfx950, for
// Q4_K, Q5_K, Q6_K, Q8_0, Q4_0, Q5_0, Q2_K and Q3_K weights.
//
// Replaces the column loop of candle-core 0.8.4 k_quants::matmul<T> (each
// output column = T::vec_dot(k, W[col], xq)) for one activation row, the
// decode call at native/arm_ai_nif/src/llama_candle.rs:119.  The integer sums
// of every block are exact; only the f32 combination order differs from
// candle's vec_dot_unopt.
//
// Mapping.  A workgroup (W = 16 wavefronts; 8 for rows of up to 8 groups) owns 56 consecutive weight rows (seven
// 8-row blocks of the row-block tile layout, so every CU of a 256-CU GPU gets
// the same bytes at the headline shape, Q4_K 14336 x 4096).  Lane l of every
// wavefront is row row0 + l (lanes 56..63 are idle); wavefront w takes the
// 256-element groups w, w + W, ...  A load instruction therefore reads piece
// p of one group for 56 rows: seven full 128-byte lines.  Because all lanes of
// a wavefront work on the same group, the activation operand of every v_dot4
// is the same for all lanes: it is read from LDS at a wave-uniform address
// (one 16-byte broadcast read per four v_dot4), so the weights are the only
// per-lane data.
//
// Schedule.  The first ceil(groups / 4) wavefronts load the activation, then
// every wavefront issues its first P weight pieces, then those wavefronts
// quantise four blocks of 256 each (Q8_K, or eight Q8_0 blocks of 32 for the
// Q8_0 / Q4_0 / Q5_0 weights; 16 lanes per 256, 16 elements per lane) into
// LDS while the weight pieces are in flight.  The 8-wavefront form with an
// f32 input instead quantises one block per wavefront (4 elements per lane),
// so that all four SIMDs take part.
// After one barrier each wavefront walks its pieces in order, keeping P of
// them in flight (compute piece j, issue piece j + P): a wavefront never
// waits at the barrier behind its own blocked load issues, and the dot
// products of the pieces that have arrived overlap the rest of the stream.
// Partial sums of a row (one per group) are added across the wavefronts
// through LDS, in wavefront order.
//
// Fewer rows (from 256; the Llama-3-8B attention projections and ffn_down,
// 4096 rows) with up to 64 groups: a workgroup owns 16 rows and lane l of a
// wavefront is row l % 16 of group phase l / 16, so one load instruction
// reads piece p of four groups for 16 rows (eight full lines) and 256
// workgroups cover 4096 rows.  The activation operand then differs between
// the four 16-lane sets of a wavefront (four broadcast LDS reads), and a
// row's partials are first added across its four lanes, then across the
// wavefronts.  From 1025 to 2048 rows, 8-row workgroups (eight group phases)
// fill the CUs instead.
#include "aq_internal.h"
#include "rl_plan.h"

namespace aq {

namespace {

constexpr int RL_ROWS = rl::ROWS56;    // weight rows per workgroup (one row per lane)
constexpr int RL_MAXG = rl::MAXG;      // groups per row (k <= 16384)
constexpr int RG_ROWS = rl::ROWS16;    // weight rows per workgroup of the four-group-phase form
constexpr int RG_MIN_N = rl::MIN_N16;  // rows from which that form is used (up to 64 groups)
constexpr int RE_ROWS = rl::ROWS8;     // weight rows per workgroup of the eight-group-phase form
constexpr int RL_NORM_MAXG = rl::NORM_MAXG;  // the fused norm: rows of up to 8192 elements (as the general matvec)

struct RlParams {
    const uint8_t *w;  // row-block tiles
    const uint16_t *wd;  // Q6_K: the d plane [n/8][ng][8] (f16)
    int64_t rb_stride;
    int n, k, ng;
    const float *x;    // fused: f32 [k]
    // fused RMSNorm (NORM): quantise rms_norm(x + xdelta) * xnorm; workgroup 0
    // writes x + xdelta to xout (xdelta, xout may be null)
    const float *xdelta, *xnorm;
    float *xout;
    float eps;
    int xf;            // RL_XF_NONE / _NORM / _SILU (see rl_body)
    ActPlanes act;     // pre-quantised planes (x null)
    float *y;
    int swiglu;        // y[4b + j] = silu(row 8b + j) * row (8b + 4 + j), j < 4
    int2 *amax;        // or null: per workgroup, (bits of the largest y, its row) over the rows it wrote
    int32_t *S, *Smin;  // [n][ng] integer dump, or null
};

// R rows per workgroup: RL_ROWS (lane = row, one group phase) or RG_ROWS
// (lane = row + 16 * group phase, four phases).  Lane (row r, phase gp) of
// wavefront w takes the groups w * GP + gp + W * GP * i, i < GPW.
//
// Q6_K (13 pieces per group: 0-7 ql, 8-11 qh, 12 the 16 int8 sub-scales; d in
// the d plane).  A lane takes the scales piece first and keeps it, and the
// qh pieces before the ql pieces that need them (the order is given at
// piece_of below); each ql piece then gives two sub-blocks' 6-bit quants
// (its nibbles and two bits of the matching qh piece).  Sums are of the
// stored quants q (0..63); candle's q - 32 is applied as -32 times the
// activation's 16-element bsum, which gives the same integers.
//
// Persistent chunks (CH; more 56-row chunks than CUs, one group per
// wavefront): a workgroup quantises the activation once and walks the chunks
// blockIdx.x, blockIdx.x + gridDim.x, ...; every piece of the next chunk is
// issued right after the same piece of the current one is consumed (P =
// pieces per group), so the stream does not drain between chunks.
//
// Input transforms of an f32 x (XF): RL_XF_NORM quantises
// rms_norm(x + delta) * w (workgroup 0 writing x + delta to xout), RL_XF_SILU
// takes x = [g (k) | u (k)] and quantises silu(g) * u, candle's
// x / (1 + e^-x) * u.
//
// The body takes its workgroup index bid of nblk, so that one launch can run
// two weights' matvecs on the same input (rl2_kernel).
template <int TYPE, int R, int W, int GPW, int P, bool EARLY, bool FUSED, bool DUMP, bool CH, int XF, bool WQ>
__device__ __forceinline__ void rl_body(const RlParams p, const int bid, const int nblk) {
    constexpr bool NORM = XF == RL_XF_NORM, SILU = XF == RL_XF_SILU;
    static_assert(XF == RL_XF_NONE || (FUSED && !DUMP), "input transforms take an f32 input and no integer dump");
    static_assert(R == RL_ROWS || R == RG_ROWS || R == RE_ROWS,
                  "56 rows, one per lane, or 16 / 8 rows in four / eight group phases");
    static_assert(TYPE == TYPE_Q4_K || TYPE == TYPE_Q5_K || TYPE == TYPE_Q6_K || TYPE == TYPE_Q8_0 ||
                  TYPE == TYPE_Q4_0 || TYPE == TYPE_Q5_0 || TYPE == TYPE_Q2_K || TYPE == TYPE_Q3_K,
                  "a type with a row-per-lane walk");
    constexpr bool Q6 = TYPE == TYPE_Q6_K, Q80 = TYPE == TYPE_Q8_0, Q5K = TYPE == TYPE_Q5_K;
    constexpr bool Q40 = TYPE == TYPE_Q4_0, Q50 = TYPE == TYPE_Q5_0, Q2K = TYPE == TYPE_Q2_K, Q3K = TYPE == TYPE_Q3_K;
    constexpr bool B16 = Q6 || Q2K || Q3K;  // bsums per 16 elements (else per 32)
    constexpr bool DP = Q6 || Q2K;          // a d plane: f16 d (Q6_K), f16 d | f16 dmin << 16 (Q2_K)
    constexpr int DB = Q2K ? 4 : 2;         // bytes per d-plane entry
    constexpr bool A80 = Q80 || Q40 || Q50;  // the activation in Q8_0 blocks of 32
    constexpr int NPG = slabs_of(TYPE);      // pieces per group
    static_assert(!CH || (R == RL_ROWS && GPW == 1 && P == NPG),
                  "persistent chunks: one group per wavefront, all its pieces in flight");
    static_assert(TYPE != TYPE_Q8_0 || (R != RL_ROWS && GPW == 1), "Q8_0: the 16- and 8-row forms");
    constexpr int GP = R == RL_ROWS ? 1 : 64 / R;  // group phases per wavefront
    __shared__ __align__(16) uint8_t xq[RL_MAXG][256];  // Q8_K quants of each group
    __shared__ __align__(16) int xb[RL_MAXG][B16 ? 16 : 8];  // bsums per 16 (Q6_K, Q2_K, Q3_K) or 32 elements
    __shared__ float xd[RL_MAXG];                       // Q8_K d
    __shared__ float xd8[A80 ? RL_MAXG : 1][8];         // Q8_0 blocks: the f16 d of each, as f32
    __shared__ int xb8[Q40 || Q50 ? RL_MAXG : 1][8];    // ... and the sum of its 32 quants
    __shared__ float red[CH ? 2 : 1][W][64];
    __shared__ float nred[W];  // NORM: the quantising wavefronts' sums of squares
    constexpr int NP = NPG * GPW;  // this wavefront's pieces, in order
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int rl = GP == 1 ? lane : lane % R, gp = GP == 1 ? 0 : lane / R;
    const int nrb = (p.n + RB - 1) / RB;
    // the rows of a chunk: this lane's row and the weight / d-plane descriptors
    struct Chunk {
        int row;
        bool rok;
        rsrc_t rw, rwd;
        uint32_t lbase, dbase;
    };
    auto chunk_at = [&](int chunk) {
        Chunk c;
        const int row0 = chunk * R;
        c.row = row0 + rl;
        c.rok = rl < R && c.row < p.n;
        const int rb0 = row0 / RB;
        // (a chunk past the rows -- which the host check rl::grid_ok
        //  keeps any launch from making -- gets an empty range, so that
        //  every load of it reads zeros: a grid larger than the chunk count
        //  would otherwise wrap rbs * rb_stride to a 4 GB range)
        const int rbs = max(0, min(R / RB, nrb - rb0));
        c.rw = buf_rsrc(p.w + (int64_t)rb0 * p.rb_stride, (uint32_t)(rbs * p.rb_stride));
        c.lbase = c.rok ? (uint32_t)((rl / RB) * p.rb_stride + (rl % RB) * 16) : BUF_OOB;
        c.rwd = buf_rsrc(DP ? (const uint8_t *)p.wd + (int64_t)rb0 * p.ng * RB * DB : nullptr,
                         DP ? (uint32_t)(rbs * p.ng * RB * DB) : 0u);
        c.dbase = c.rok ? (uint32_t)(((rl / RB) * p.ng * RB + (rl % RB)) * DB) : BUF_OOB;
        return c;
    };
    Chunk cur = chunk_at(bid);
    auto group_of = [&](int j) { return wave * GP + gp + W * GP * (j / NPG); };
    // the piece a lane reads at its j-th step within a group
    // (Q6_K: 12, 8, 9, 0-3, 10, 11, 4-7 in the 56-row form, which holds two
    //  qh pieces at a time; 12, 8-11, 0-7 in the 16-row form, where that
    //  order measured fewer registers)
    constexpr bool HALVES = R == RL_ROWS;
    auto piece_of = [&](int pc) {
        // the eight d of a Q8_0 / Q4_0 / Q5_0 group first (Q5_0: then its two
        // qh pieces), then the quants in order
        if (Q80) return pc == 0 ? 16 : pc - 1;
        if (Q40) return pc == 0 ? 8 : pc - 1;
        if (Q50) return pc == 0 ? 10 : pc < 3 ? 7 + pc : pc - 3;
        if (Q3K) return pc == 0 ? 6 : pc - 1;  // scales and d, hmask, then qs
        if (!Q6) return pc;
        if (!HALVES) return pc == 0 ? 12 : pc < 5 ? 7 + pc : pc - 5;
        return pc == 0 ? 12 : pc < 3 ? 7 + pc : pc < 7 ? pc - 3 : pc < 9 ? 3 + pc : pc - 5;
    };

    uint4 ring[P];
    uint32_t dring[GPW];  // Q6_K: the f16 d of each of this lane's groups
    // (on = false: an out-of-range load that returns zeros, in place of a branch)
    auto issue_in = [&](const Chunk &c, int j, bool on) {
        const int g = group_of(j);
        const bool ok = on && g < p.ng;
        const uint32_t off = ok ? c.lbase + (uint32_t)((g * NPG + piece_of(j % NPG)) * 128) : BUF_OOB;
        const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(c.rw, off, 0, BUF_NT);
        ring[j % P] = make_uint4(t.x, t.y, t.z, t.w);
        if (DP && j % NPG == 0) {
            const uint32_t doff = ok ? c.dbase + (uint32_t)(g * RB * DB) : BUF_OOB;
            dring[j / NPG] = Q2K ? __builtin_amdgcn_raw_buffer_load_b32(c.rwd, doff, 0, BUF_NT)
                                 : __builtin_amdgcn_raw_buffer_load_b16(c.rwd, doff, 0, BUF_NT);
        }
    };
    auto issue = [&](int j) { issue_in(cur, j, true); };

    // 1. the activation's loads: wavefront w < ceil(ng / 4) stages blocks
    //    4w .. 4w + 3, 16 lanes (s = lane & 15) per block, or (WIDE: an f32
    //    input in a form launched with a wavefront for every block, WQ)
    //    wavefront w < ng block w, lane l its elements 4l .. 4l + 3; then (EARLY) this
    //    wavefront's first P weight pieces, so that they are in flight while
    //    the activation is quantised (the loads are waited for in issue
    //    order).  With most wavefronts quantising (the 16-wavefront form),
    //    issuing only the first piece before the quantisation and the rest
    //    after it measured faster than either all before or all after.
    //    WQ is taken by the 8-wavefront 56-row form (rows of up to 8
    //    groups), where 16-lane quantisers would leave two of the four SIMDs
    //    idle; in the 16-wavefront form the four 16-lane quantisers already
    //    take one SIMD each, and 64-lane blocks measured slower there (the
    //    headline 7.5 against 6.7 us), as did eight such wavefronts in place
    //    of two in the 16- and 8-row forms.
    static_assert(!WQ || GPW == 1, "one block per wavefront: one group per wavefront");
    constexpr bool WIDE = FUSED && WQ;  // the host checks ng <= W
    constexpr int NV = WIDE ? 4 : 16;  // activation values per lane
    const int s = lane & 15;
    const int gb = WIDE ? wave : 4 * wave + (lane >> 4);
    const bool quantiser = WIDE ? wave < p.ng : wave < (p.ng + 3) / 4;  // uniform
    const bool gbok = gb < p.ng;
    u32x4 xv[4], dv[4], nv[4];
    uint32_t xbs = 0, xdb = 0;
    const uint32_t xo = gbok ? (uint32_t)((gb * QK_K + (WIDE ? 4 * lane : 16 * s)) * 4) : BUF_OOB;
    if (quantiser) {
        if (FUSED) {
            const rsrc_t rx = buf_rsrc(p.x, (uint32_t)(p.k * 4));
#pragma unroll
            for (int i = 0; i < NV / 4; i++) xv[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 16 * i, 0, 0);
            if (NORM) {  // a null delta: an empty range, zeros
                const rsrc_t rdl = buf_rsrc(p.xdelta, p.xdelta ? (uint32_t)(p.k * 4) : 0u);
                const rsrc_t rnw = buf_rsrc(p.xnorm, (uint32_t)(p.k * 4));
#pragma unroll
                for (int i = 0; i < NV / 4; i++) {
                    dv[i] = __builtin_amdgcn_raw_buffer_load_b128(rdl, xo + 16 * i, 0, 0);
                    nv[i] = __builtin_amdgcn_raw_buffer_load_b128(rnw, xo + 16 * i, 0, 0);
                }
            } else if (SILU) {  // u = the second half of x
                const rsrc_t ru = buf_rsrc(p.x + p.k, (uint32_t)(p.k * 4));
#pragma unroll
                for (int i = 0; i < NV / 4; i++) dv[i] = __builtin_amdgcn_raw_buffer_load_b128(ru, xo + 16 * i, 0, 0);
            }
        } else {
            const rsrc_t rq = buf_rsrc(p.act.qs, (uint32_t)p.k);
            const rsrc_t rs = buf_rsrc(p.act.bsums, (uint32_t)((p.k / 16) * 2));
            const rsrc_t rd = buf_rsrc(p.act.d, (uint32_t)((p.k / (A80 ? QK8_0 : QK_K)) * 4));
            xv[0] = __builtin_amdgcn_raw_buffer_load_b128(rq, gbok ? (uint32_t)(gb * QK_K + 16 * s) : BUF_OOB, 0, 0);
            if (!A80)
                xbs = __builtin_amdgcn_raw_buffer_load_b16(rs, gbok ? (uint32_t)((gb * 16 + s) * 2) : BUF_OOB, 0, 0);
            // Q8_0 blocks: d of block 8 gb + s / 2 (the two lanes of a block read the same)
            const uint32_t dof = A80 ? (uint32_t)((gb * 8 + (s >> 1)) * 4) : (uint32_t)(gb * 4);
            xdb = __builtin_amdgcn_raw_buffer_load_b32(rd, gbok ? dof : BUF_OOB, 0, 0);
        }
    }
    {
#pragma unroll
        for (int j = 0; j < (EARLY ? P : 1) && j < NP; j++) issue(j);
    }
    // 2. quantise (or unpack) into LDS, then one barrier (LDS writes only).
    //    NORM: h = x + delta and the row's sum of squares first (every
    //    wavefront takes the barrier; lanes past the row hold zeros), then
    //    (h * (1 / sqrt(mean(h^2) + eps))) * w is quantised.
    float v[NV];
    if (FUSED && quantiser) {
#pragma unroll
        for (int i = 0; i < NV / 4; i++) {
            v[4 * i] = u32_as_f32(xv[i].x);
            v[4 * i + 1] = u32_as_f32(xv[i].y);
            v[4 * i + 2] = u32_as_f32(xv[i].z);
            v[4 * i + 3] = u32_as_f32(xv[i].w);
        }
    }
    if (SILU && quantiser) {
        float uv[NV];
#pragma unroll
        for (int i = 0; i < NV / 4; i++) {
            uv[4 * i] = u32_as_f32(dv[i].x);
            uv[4 * i + 1] = u32_as_f32(dv[i].y);
            uv[4 * i + 2] = u32_as_f32(dv[i].z);
            uv[4 * i + 3] = u32_as_f32(dv[i].w);
        }
#pragma unroll
        for (int i = 0; i < NV; i++) v[i] = (v[i] / (1.0f + expf(-v[i]))) * uv[i];
    }
    if (NORM) {
        float ss = 0.0f;
        if (quantiser) {
#pragma unroll
            for (int i = 0; i < NV / 4; i++) {
                v[4 * i] += u32_as_f32(dv[i].x);
                v[4 * i + 1] += u32_as_f32(dv[i].y);
                v[4 * i + 2] += u32_as_f32(dv[i].z);
                v[4 * i + 3] += u32_as_f32(dv[i].w);
            }
#pragma unroll
            for (int i = 0; i < NV; i++) ss = __builtin_fmaf(v[i], v[i], ss);
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
            if (lane == 0) nred[wave] = ss;
        }
        lds_barrier();
        if (quantiser) {
            const int nq = WIDE ? p.ng : (p.ng + 3) / 4;
            float tot = 0.0f;
            for (int w2 = 0; w2 < nq; w2++) tot += nred[w2];
            const float mden = sqrtf(tot / (float)p.k + p.eps);
            if (p.xout && bid == 0 && gbok) {  // the residual stream x + delta
#pragma unroll
                for (int i = 0; i < NV / 4; i++)
                    *(float4 *)(p.xout + gb * QK_K + (WIDE ? 4 * lane : 16 * s) + 4 * i) =
                        make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
            }
            // candle's h / m as h * (1 / m): one division per lane, not 16
            // (within one rounding of the quotient; the reordered sum of
            // squares already moves m by as much)
            const float rm = 1.0f / mden;
#pragma unroll
            for (int i = 0; i < NV / 4; i++) {
                v[4 * i] = (v[4 * i] * rm) * u32_as_f32(nv[i].x);
                v[4 * i + 1] = (v[4 * i + 1] * rm) * u32_as_f32(nv[i].y);
                v[4 * i + 2] = (v[4 * i + 2] * rm) * u32_as_f32(nv[i].z);
                v[4 * i + 3] = (v[4 * i + 3] * rm) * u32_as_f32(nv[i].w);
            }
        }
    }
    if constexpr (WIDE) {
        if (quantiser) {
            // lane l: quants 4l .. 4l + 3 of block gb; the 8 lanes of a 32-element
            // sub-block (a Q8_0 block) are one half-row, the 4 of a 16-element one a quad
            if (A80) {
                uint16_t d16;
                const uint32_t qv = q8_0_block_8lanes(v, &d16);
                int bsum = sdot4((int)qv, 0x01010101, 0);
                bsum += dpp_i<DPP_QUAD_XOR1>(bsum);
                bsum += dpp_i<DPP_QUAD_XOR2>(bsum);
                bsum += dpp_i<DPP_HALF_MIRROR>(bsum);
                *(uint32_t *)&xq[gb][4 * lane] = qv;
                if ((lane & 7) == 0) {
                    xd8[gb][lane >> 3] = f16_bits_to_f32(d16);
                    if (Q40 || Q50) xb8[gb][lane >> 3] = bsum;
                }
            } else {
                int bsum;  // this quad's 16 quants
                float d;
                const uint32_t qv = q8k_block_wave(v, lane, &bsum, &d);
                const int pair = bsum + dpp_i<DPP_HALF_MIRROR>(bsum);  // and the other quad of the half-row
                *(uint32_t *)&xq[gb][4 * lane] = qv;
                if (B16) {
                    if ((lane & 3) == 0) xb[gb][lane >> 2] = bsum;
                } else if ((lane & 7) == 0) {
                    xb[gb][lane >> 3] = pair;
                }
                if (lane == 0) xd[gb] = d;
            }
        }
    } else if (quantiser) {
        uint4 qv;
        int bsum;
        float d;
        if (FUSED && A80) {
            uint16_t d16;
            qv = q8_0_block_2lanes(v, &d16);
            d = f16_bits_to_f32(d16);
            bsum = 0;
        } else if (FUSED) {
            qv = q8k_block_row16(v, s, &bsum, &d);
        } else {
            qv = make_uint4(xv[0].x, xv[0].y, xv[0].z, xv[0].w);
            bsum = (int)(int16_t)xbs;
            d = u32_as_f32(xdb);
        }
        if (Q40 || Q50) {  // a Q8_0 block's quant sum: this lane's 16, then the pair's
            bsum = sdot4((int)qv.x, 0x01010101, 0);
            bsum = sdot4((int)qv.y, 0x01010101, bsum);
            bsum = sdot4((int)qv.z, 0x01010101, bsum);
            bsum = sdot4((int)qv.w, 0x01010101, bsum);
        }
        const int pair = bsum + dpp_i<DPP_QUAD_XOR1>(bsum);  // sub-block s/2 (two 16-element halves)
        if (gbok) {
            *(uint4 *)&xq[gb][16 * s] = qv;
            if (A80) {
                if ((s & 1) == 0) {
                    xd8[gb][s >> 1] = d;
                    if (Q40 || Q50) xb8[gb][s >> 1] = pair;
                }
            } else {
                if (B16) xb[gb][s] = bsum;
                else if ((s & 1) == 0) xb[gb][s >> 1] = pair;
                if (s == 0) xd[gb] = d;
            }
        }
    }
    if (!EARLY) {
#pragma unroll
        for (int j = 1; j < P && j < NP; j++) issue(j);
    }
    lds_barrier();

    // 3. walk the pieces: piece 0 of a group = d, dmin, 12 scale bytes; piece
    //    1 + 2c + h = qs bytes 32c + 16h .. +15 (low nibbles: elements
    //    64c + 16h + i of sub-block 2c; high: 64c + 32 + 16h + i of 2c + 1)
    const int nch = (p.n + R - 1) / R;
    // (amax: this lane's largest value so far and its row -- the first of
    //  equal values; a NaN never wins)
    float abv = -INFINITY;
    int abi = 0x7fffffff;
    for (int chunk = bid, it = 0;; it++) {  // one chunk unless CH
    const int nextc = chunk + nblk;
    const bool more = CH && nextc < nch;  // uniform
    Chunk nxt = cur;
    if (more) nxt = chunk_at(nextc);
    const int row = cur.row;
    const bool rok = cur.rok;
    float f = 0.0f;
    uint32_t dwq = 0;  // Q6_K: this group's d (taken before the next chunk's load reuses the slot)
    int bs[8];
    float dx = 0.0f;
    uint32_t sc03 = 0, sc47 = 0, mn03 = 0, mn47 = 0, dwp = 0;
    uint4 qhr[4] = {};  // Q6_K: the qh pieces held (HALVES: those of the current 128-element half)
    uint4 sc6 = {};     // Q6_K: the group's 16 sub-scales
    int S = 0, il = 0, ih = 0;
    // a group's terms that need only its piece 0 and the activation, taken
    // when piece 0 arrives rather than after its last piece: d_w * d_x, and
    // (Q4_K, Q5_K, Q2_K) the min sum and (dmin_w * d_x) * smin
    int smin = 0;
    float dwdx = 0.0f, fmin = 0.0f;
    // (a wavefront without a group -- those that only quantise, e.g. three of
    //  the six at 22 groups in the 8-row form -- skips the walk as a whole:
    //  its out-of-range loads and zero sums cost w2 of the decode step about
    //  0.4-1.0 us; persistent, the pieces in flight across chunks then have
    //  one path through it)
    if (wave * GP < p.ng) {  // uniform: the wavefront's first group (its phase 0)
    #pragma unroll
        for (int j = 0; j < NP; j++) {
            const int pc = j % NPG;
            const int g = group_of(j);
            if (GP == 1 && !CH && g >= p.ng) break;  // uniform
            const bool gok = g < p.ng;         // (lanes of several phases: per lane)
            const int gl = gok ? g : 0;        // a group whose LDS entries are written
            const uint4 q = ring[j % P];
            if (Q80) {
                // piece 0: the eight blocks' f16 d (kept in sc6); piece 1 + i:
                // quants 16i .. 16i + 15, the half i & 1 of block i / 2, whose
                // dot closes as candle's ((isum * d_w) * d_x)
                if (pc == 0) {
                    sc6 = q;
                } else {
                    const int i = pc - 1, jb = i >> 1;
                    const int4 xv4 = *(const int4 *)&xq[gl][16 * i];
                    if ((i & 1) == 0) il = 0;
                    il = sdot4((int)q.x, xv4.x, il);
                    il = sdot4((int)q.y, xv4.y, il);
                    il = sdot4((int)q.z, xv4.z, il);
                    il = sdot4((int)q.w, xv4.w, il);
                    if (i & 1) {
                        const uint32_t dws[4] = {sc6.x, sc6.y, sc6.z, sc6.w};
                        const float dw = f16_bits_to_f32(dws[jb >> 1] >> (16 * (jb & 1)));
                        if (gok) f += ((float)il * dw) * xd8[gl][jb];
                        if (DUMP && rok && gok) {  // per 32-element block (k is a multiple of 256)
                            p.S[(int64_t)row * (8 * p.ng) + 8 * g + jb] = il;
                            p.Smin[(int64_t)row * (8 * p.ng) + 8 * g + jb] = 0;
                        }
                    }
                }
            } else if (Q40 || Q50) {
                // piece 0: the eight f16 d (kept in sc6); Q5_0: pieces 1, 2: the
                // 32-bit qh of blocks 0-3, 4-7; then block jb per piece: low
                // nibbles elements 0..15, high nibbles 16..31, value q - 8
                // (Q5_0: bit e of qh at bit 4, value q - 16).  candle's
                // ((isum * d_w) * d_x), isum = sum q*qx - 8 (16) * sum qx
                constexpr int QB = Q50 ? 3 : 1;  // the first quant piece
                if (pc == 0) {
                    sc6 = q;
                } else if (Q50 && pc < QB) {
                    qhr[pc - 1] = q;
                } else {
                    const int jb = pc - QB;
                    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
                    uint32_t hq = 0;
                    if (Q50) {
                        const uint4 hh = qhr[jb >> 2];
                        const uint32_t hw[4] = {hh.x, hh.y, hh.z, hh.w};
                        hq = hw[jb & 3];
                    }
                    const int4 x0 = *(const int4 *)&xq[gl][32 * jb], x1 = *(const int4 *)&xq[gl][32 * jb + 16];
                    const int x0v[4] = {x0.x, x0.y, x0.z, x0.w}, x1v[4] = {x1.x, x1.y, x1.z, x1.w};
                    int isum = 0;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        uint32_t lo = qw[i] & 0x0F0F0F0Fu, hi = (qw[i] >> 4) & 0x0F0F0F0Fu;
                        if (Q50) {
                            lo |= spread4((hq >> (4 * i)) & 0xFu);
                            hi |= spread4((hq >> (16 + 4 * i)) & 0xFu);
                        }
                        isum = sdot4((int)lo, x0v[i], isum);
                        isum = sdot4((int)hi, x1v[i], isum);
                    }
                    isum -= (Q50 ? 16 : 8) * xb8[gl][jb];
                    const uint32_t dws[4] = {sc6.x, sc6.y, sc6.z, sc6.w};
                    const float dw = f16_bits_to_f32(dws[jb >> 1] >> (16 * (jb & 1)));
                    if (gok) f += ((float)isum * dw) * xd8[gl][jb];
                    if (DUMP && rok && gok) {  // per 32-element block (k is a multiple of 256)
                        p.S[(int64_t)row * (8 * p.ng) + 8 * g + jb] = isum;
                        p.Smin[(int64_t)row * (8 * p.ng) + 8 * g + jb] = 0;
                    }
                }
            } else if (Q2K) {
                // piece 0: scale | min << 4 of the 16 16-element groups (kept in
                // sc6); piece 1 + 2hf + t: qs bytes 32hf + 16t .., whose bits
                // 2jj, 2jj + 1 are elements 128hf + 32jj + 16t + i (group
                // 8hf + 2jj + t)
                if (pc == 0) {
                    sc6 = q;
                    dx = xd[gl];
                    dwq = dring[j / NPG];
                    S = 0;
                    smin = 0;
                    const uint32_t scw[4] = {sc6.x, sc6.y, sc6.z, sc6.w};
#pragma unroll
                    for (int gq = 0; gq < 16; gq++) smin += (int)((scw[gq >> 2] >> (8 * (gq & 3) + 4)) & 15u) * xb[gl][gq];
                    const float dw = f16_bits_to_f32(dwq), dmw = f16_bits_to_f32(dwq >> 16);
                    dwdx = dw * dx;
                    fmin = (dmw * dx) * (float)smin;
                } else {
                    const int hf = (pc - 1) >> 1, t = (pc - 1) & 1;
                    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
                    const uint32_t scw[4] = {sc6.x, sc6.y, sc6.z, sc6.w};
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) {
                        const int grp = 8 * hf + 2 * jj + t;
                        const int4 xv4 = *(const int4 *)&xq[gl][128 * hf + 32 * jj + 16 * t];
                        const int xa[4] = {xv4.x, xv4.y, xv4.z, xv4.w};
                        int is = 0;
#pragma unroll
                        for (int i = 0; i < 4; i++) is = sdot4((int)((qw[i] >> (2 * jj)) & 0x03030303u), xa[i], is);
                        S += (int)((scw[grp >> 2] >> (8 * (grp & 3))) & 15u) * is;
                    }
                }
            } else if (Q3K) {
                // piece 0: scales[12] then the f16 d; pieces 1, 2: hmask bytes
                // 0..15, 16..31 (kept); piece 3 + 2hf + t: qs bytes 32hf + 16t ..
                // with the elements as Q2_K's, value (the two bits | hmask bit
                // 4hf + jj << 2) - 4, taken as the group's bsum times 4; the
                // 6-bit group scale (candle's auxs form) - 32
                if (pc == 0) {
                    const uint32_t a0 = q.x, a1 = q.y, tmp = q.z;
                    sc6 = make_uint4((a0 & 0x0F0F0F0Fu) | ((tmp & 0x03030303u) << 4),
                                     (a1 & 0x0F0F0F0Fu) | (((tmp >> 2) & 0x03030303u) << 4),
                                     ((a0 >> 4) & 0x0F0F0F0Fu) | (((tmp >> 4) & 0x03030303u) << 4),
                                     ((a1 >> 4) & 0x0F0F0F0Fu) | (((tmp >> 6) & 0x03030303u) << 4));
                    dwq = q.w;
                    dx = xd[gl];
                    dwdx = f16_bits_to_f32(dwq) * dx;
                    S = 0;
                } else if (pc < 3) {
                    qhr[pc - 1] = q;
                } else {
                    const int hf = (pc - 3) >> 1, t = (pc - 3) & 1;
                    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
                    const uint4 hb = qhr[t];
                    const uint32_t hv[4] = {hb.x, hb.y, hb.z, hb.w};
                    const uint32_t scw[4] = {sc6.x, sc6.y, sc6.z, sc6.w};
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) {
                        const int grp = 8 * hf + 2 * jj + t;
                        const int4 xv4 = *(const int4 *)&xq[gl][128 * hf + 32 * jj + 16 * t];
                        const int xa[4] = {xv4.x, xv4.y, xv4.z, xv4.w};
                        int is = 0;
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const uint32_t u = ((qw[i] >> (2 * jj)) & 0x03030303u) |
                                               (((hv[i] >> (4 * hf + jj)) & 0x01010101u) << 2);
                            is = sdot4((int)u, xa[i], is);
                        }
                        S += ((int)((scw[grp >> 2] >> (8 * (grp & 3))) & 0xffu) - 32) * (is - 4 * xb[gl][grp]);
                    }
                }
            } else if (Q6) {
                if (pc == 0) {
                    sc6 = q;
                    dx = xd[gl];
                    dwq = dring[j / NPG];
                    dwdx = f16_bits_to_f32(dwq) * dx;
                    S = 0;
                } else if (HALVES ? (pc == 1 || pc == 2 || pc == 7 || pc == 8) : pc < 5) {
                    qhr[HALVES ? (pc - 1) % 2 : pc - 1] = q;
                } else {
                    // ql piece 4n + c: low nibbles are elements 128n + 16c + i
                    // (sub-block 8n + c), high nibbles 128n + 64 + 16c + i
                    // (sub-block 8n + 4 + c); their top two bits are bits
                    // 2(c >> 1) and 2(c >> 1) + 4 of qh[32n + 16(c & 1) + i]
                    const int ip = HALVES && pc < 7 ? pc - 3 : pc - 5, n = ip >> 2, c = ip & 3;
                    const uint4 h = qhr[HALVES ? c & 1 : 2 * n + (c & 1)];
                    const int sl = 2 * (c >> 1), jl = 8 * n + c, jh = jl + 4;
                    const int4 xl = *(const int4 *)&xq[gl][16 * jl];
                    const int4 xh = *(const int4 *)&xq[gl][16 * jh];
                    auto lo = [&](uint32_t v, uint32_t hb) { return (int)((v & 0x0F0F0F0Fu) | (((hb >> sl) & 0x03030303u) << 4)); };
                    auto hi = [&](uint32_t v, uint32_t hb) {
                        return (int)(((v >> 4) & 0x0F0F0F0Fu) | (((hb >> (sl + 4)) & 0x03030303u) << 4));
                    };
                    int a = 0, b = 0;
                    a = sdot4(lo(q.x, h.x), xl.x, a);
                    b = sdot4(hi(q.x, h.x), xh.x, b);
                    a = sdot4(lo(q.y, h.y), xl.y, a);
                    b = sdot4(hi(q.y, h.y), xh.y, b);
                    a = sdot4(lo(q.z, h.z), xl.z, a);
                    b = sdot4(hi(q.z, h.z), xh.z, b);
                    a = sdot4(lo(q.w, h.w), xl.w, a);
                    b = sdot4(hi(q.w, h.w), xh.w, b);
                    const uint32_t scw[4] = {sc6.x, sc6.y, sc6.z, sc6.w};
                    const int scl = (int)(int8_t)((scw[jl >> 2] >> (8 * (jl & 3))) & 0xffu);
                    const int sch = (int)(int8_t)((scw[jh >> 2] >> (8 * (jh & 3))) & 0xffu);
                    S += scl * (a - 32 * xb[gl][jl]) + sch * (b - 32 * xb[gl][jh]);
                }
            } else if (pc == 0) {
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
                smin = 0;
#pragma unroll
                for (int jj = 0; jj < 8; jj++) smin += (int)(((jj < 4 ? mn03 : mn47) >> (8 * (jj & 3))) & 0xffu) * bs[jj];
                const float dw = f16_bits_to_f32(dwp), dmw = f16_bits_to_f32(dwp >> 16);
                dwdx = dw * dx;
                fmin = (dmw * dx) * (float)smin;
            } else if (Q5K && pc < 3) {
                qhr[pc - 1] = q;  // qh bytes 0..15, 16..31
            } else {
                // qs piece 1 + 2c + h (Q5_K: 3 + 2c + h)
                const int c = (pc - (Q5K ? 3 : 1)) >> 1, h = (pc - (Q5K ? 3 : 1)) & 1;
                // x of the low nibbles (elements 64c + 16h ..) and of the high
                // nibbles (64c + 32 + 16h ..): the same for every lane
                const int4 xl = *(const int4 *)&xq[gl][64 * c + 16 * h];
                const int4 xh = *(const int4 *)&xq[gl][64 * c + 32 + 16 * h];
                if (h == 0) il = ih = 0;
                const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
                uint32_t hw[4] = {0u, 0u, 0u, 0u};
                if (Q5K) {  // qh bytes 16h + i: bit 2c for the low nibble's element, 2c + 1 for the high
                    const uint4 hb = qhr[h];
                    hw[0] = hb.x;
                    hw[1] = hb.y;
                    hw[2] = hb.z;
                    hw[3] = hb.w;
                }
                const int xlv[4] = {xl.x, xl.y, xl.z, xl.w}, xhv[4] = {xh.x, xh.y, xh.z, xh.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    // Q4_K: the high nibbles in place, (q & 0xF0) ^ 0x80 = 16 q - 128 as
                    // a signed byte (one three-input bit operation)
                    uint32_t lo = qw[i] & 0x0F0F0F0Fu;
                    uint32_t hi = Q5K ? (qw[i] >> 4) & 0x0F0F0F0Fu : (qw[i] & 0xF0F0F0F0u) ^ 0x80808080u;
                    if (Q5K) {
                        lo |= ((hw[i] >> (2 * c)) & 0x01010101u) << 4;
                        hi |= ((hw[i] >> (2 * c + 1)) & 0x01010101u) << 4;
                    }
                    il = sdot4((int)lo, xlv[i], il);
                    ih = sdot4((int)hi, xhv[i], ih);
                }
                if (h == 1) {
                    // Q4_K: sum q x = (sum (16 q - 128) x + 128 sum x) / 16, exactly
                    if (!Q5K) ih = (ih + 128 * bs[2 * c + 1]) >> 4;
                    const uint32_t sw = c < 2 ? sc03 : sc47;
                    S += (int)((sw >> (16 * (c & 1))) & 0xffu) * il + (int)((sw >> (16 * (c & 1) + 8)) & 0xffu) * ih;
                }
            }
            if (j + P < NP) issue(j + P);
            else if (CH) {
                issue_in(nxt, j + P - NP, more);
                __builtin_amdgcn_sched_barrier(0);  // keep the next chunk's load behind this piece's use
            }
            if (!A80 && pc == NPG - 1) {
                // (d_w * d_x) * S - (dmin_w * d_x) * smin (Q4_K, Q5_K, Q2_K),
                // (d_w * d_x) * S (Q6_K, Q3_K)
                constexpr bool MIN = !(Q6 || Q3K);
                if (gok) {
                    if (MIN) f += dwdx * (float)S - fmin;
                    else f += dwdx * (float)S;
                }
                if (DUMP && rok && gok) {
                    p.S[(int64_t)row * p.ng + g] = S;
                    p.Smin[(int64_t)row * p.ng + g] = MIN ? smin : 0;
                }
            }
        }
    }
    // 4. the row's partials: over its group phases within the wavefront,
    //    then over the wavefronts, in wavefront order
    if (GP == 8) f += __shfl_xor(f, 8);
    if (GP >= 4) f += __shfl_xor(f, 16);
    if (GP >= 2) f += __shfl_xor(f, 32);
    red[CH ? it & 1 : 0][wave][lane] = f;
    lds_barrier();
    if (p.swiglu) {  // uniform
        // every lane of wavefront 0 holds the sum of row (its lane mod R);
        // an 8-row block's gate rows 0-3 take their up rows 4-7 four lanes
        // on, and write candle's silu(g) * u = (g / (1 + e^-g)) * u
        if (wave == 0) {
            float t = 0.0f;
#pragma unroll
            for (int w = 0; w < W; w++) t += red[CH ? it & 1 : 0][w][lane];
            const float u = __shfl_down(t, 4);
            if (rok && gp == 0 && (row & 4) == 0) p.y[(row >> 3) * 4 + (row & 3)] = (t / (1.0f + expf(-t))) * u;
        }
    } else if (wave == 0) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) t += red[CH ? it & 1 : 0][w][lane];
        if (rok && gp == 0) {
            p.y[row] = t;
            if (t > abv || (t == abv && row < abi)) {
                abv = t;
                abi = row;
            }
        }
    }
    if (!more) break;  // uniform
    chunk = nextc;
    cur = nxt;
    }
    if (p.amax && wave == 0) {  // uniform: the workgroup's largest value and its row
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const float ov = __shfl_xor(abv, o);
            const int oi = __shfl_xor(abi, o);
            if (ov > abv || (ov == abv && oi < abi)) {
                abv = ov;
                abi = oi;
            }
        }
        if (lane == 0) p.amax[bid] = make_int2((int)f32_as_u32(abv), abi);
    }
}

template <int TYPE, int R, int W, int GPW, int P, bool EARLY, bool FUSED, bool DUMP, bool CH = false, int XF = RL_XF_NONE,
          bool WQ = false>
__global__ __launch_bounds__(W * 64) void rl_kernel(RlParams p) {
    rl_body<TYPE, R, W, GPW, P, EARLY, FUSED, DUMP, CH, XF, WQ>(p, (int)blockIdx.x, (int)gridDim.x);
}

// Two weights on the same f32 input in one launch (the decode step's wq|wk
// and wv): workgroups [0, g1) take the first, the rest the second; both in
// the form of R (16 or 8) rows with W wavefronts (their LDS is separate).
// A wavefront past the groups adds 0 to its rows, so W wavefronts give the
// same sums as a single weight's launch with fewer.
template <int T1, int T2, int R, int W, int XF, bool WQ>
__global__ __launch_bounds__(W * 64) void rl2_kernel(RlParams p1, RlParams p2, int g1) {
    constexpr int P1 = T1 == TYPE_Q6_K ? 13 : 9, P2 = T2 == TYPE_Q6_K ? 13 : 9;
    const int bid = (int)blockIdx.x;
    if (bid < g1) rl_body<T1, R, W, 1, P1, true, true, false, false, XF, WQ>(p1, bid, g1);  // uniform
    else rl_body<T2, R, W, 1, P2, true, true, false, false, XF, WQ>(p2, bid - g1, (int)gridDim.x - g1);
}

template <int TYPE, int R, int W, int GPW, int P, bool EARLY, bool CH = false, bool WQ = false>
hipError_t launch_g(const RlParams &p, unsigned grid, bool fused, bool dump, hipStream_t s) {
    // one workgroup per chunk (persistent: at most one per chunk), never a
    // workgroup past the weight's rows
    if (!rl::grid_ok(R, p.n, grid, CH)) return hipErrorInvalidValue;
    // one group per wavefront: a wavefront for every group; WQ: a wavefront
    // for every block (an f32 input is quantised block w in wavefront w)
    if (((R == RL_ROWS && GPW == 1) || WQ) && p.ng > W) return hipErrorInvalidValue;
    if (p.xf == RL_XF_NORM) {  // input transforms: f32 input, no dump (the caller checks)
        rl_kernel<TYPE, R, W, GPW, P, EARLY, true, false, CH, RL_XF_NORM, WQ><<<grid, W * 64, 0, s>>>(p);
        return hipGetLastError();
    }
    if (p.xf == RL_XF_SILU) {
        rl_kernel<TYPE, R, W, GPW, P, EARLY, true, false, CH, RL_XF_SILU, WQ><<<grid, W * 64, 0, s>>>(p);
        return hipGetLastError();
    }
    if (fused) {
        if (dump) rl_kernel<TYPE, R, W, GPW, P, EARLY, true, true, CH, RL_XF_NONE, WQ><<<grid, W * 64, 0, s>>>(p);
        else rl_kernel<TYPE, R, W, GPW, P, EARLY, true, false, CH, RL_XF_NONE, WQ><<<grid, W * 64, 0, s>>>(p);
    } else {
        if (dump) rl_kernel<TYPE, R, W, GPW, P, EARLY, false, true, CH><<<grid, W * 64, 0, s>>>(p);
        else rl_kernel<TYPE, R, W, GPW, P, EARLY, false, false, CH><<<grid, W * 64, 0, s>>>(p);
    }
    return hipGetLastError();
}

bool rows56(int type, int64_t n, int ng) { return rl::wide(type == TYPE_Q6_K, type == TYPE_Q8_0, n, ng); }
}  // namespace

int rowlane_grid(int type, int64_t n, int64_t k) {
    return (int)rl::plan(type == TYPE_Q6_K, type == TYPE_Q8_0, n, (int)(k / QK_K)).grid;
}

namespace {
bool rows8(int64_t n, int ng) { return rl::narrow8(n, ng); }

// The launch shapes of one weight type (pieces in flight: P; 16 wavefronts
// with six Q4_K pieces in flight measured fastest at the headline, one group
// per wavefront; longer rows take two groups each)
template <int TYPE>
hipError_t launch_type(const RlParams &p, int64_t n, int ng, bool wide, bool fused, bool dump, hipStream_t s) {
    constexpr bool Q6 = TYPE == TYPE_Q6_K, Q80 = TYPE == TYPE_Q8_0;
    constexpr int NPG = slabs_of(TYPE);  // 9 (Q4_K, Q4_0), 11 (Q5_K, Q5_0), 13 (Q6_K), 17 (Q8_0)
    const rl::Plan pl = rl::plan(Q6, Q80, n, ng);
    const unsigned grid = pl.grid;
    if constexpr (!Q80) if (wide) {
        // more chunks than CUs: persistent workgroups, one per CU
        // (one wavefront per group: 8 wavefronts for up to 8 groups, where
        //  the other 8 of 16 would only wait)
        if (ng <= 8 && pl.persistent) return launch_g<TYPE, RL_ROWS, 8, 1, NPG, true, true, true>(p, grid, fused, dump, s);
        if (ng <= 16 && pl.persistent) return launch_g<TYPE, RL_ROWS, 16, 1, NPG, true, true>(p, grid, fused, dump, s);
        if (ng <= 8) return launch_g<TYPE, RL_ROWS, 8, 1, Q6 ? 8 : NPG == 11 ? 7 : 6, true, false, true>(p, grid, fused, dump, s);
        if (ng <= 16) return launch_g<TYPE, RL_ROWS, 16, 1, Q6 ? 8 : NPG == 11 ? 7 : 6, true>(p, grid, fused, dump, s);
        if constexpr (!Q6) return launch_g<TYPE, RL_ROWS, 16, 2, 12, true>(p, grid, fused, dump, s);
        return hipErrorNotSupported;
    }
    // 16 rows: as many wavefronts as four groups each need (every lane one
    // group; two for up to 8 groups, where a third and fourth wavefront
    // would only quantise and wait: 7 % faster at 5632 x 2048, and eight
    // quantising one block each measured slower still); the quantising
    // wavefronts (four blocks each) are then always enough.  Up to 32 groups all of a lane's pieces are in flight from the
    // start; with 12-16 wavefronts (ffn_down, 56 groups: 14) six (seven for
    // the 11- and 13-piece types), the first issued before the quantisation
    // and the rest after it, measured fastest.
    if (pl.rows == RE_ROWS) {
        // 8 rows: a wavefront covers eight groups, and there are as many
        // wavefronts as the quantisation needs (four blocks each); those past
        // the groups skip the walk
        if (ng <= 8) return launch_g<TYPE, RE_ROWS, 2, 1, NPG, true>(p, grid, fused, dump, s);
        if (ng <= 16) return launch_g<TYPE, RE_ROWS, 4, 1, NPG, true>(p, grid, fused, dump, s);
        if (ng <= 24) return launch_g<TYPE, RE_ROWS, 6, 1, NPG, true>(p, grid, fused, dump, s);
        return launch_g<TYPE, RE_ROWS, 8, 1, NPG, true>(p, grid, fused, dump, s);
    }
    // (a grid of at most 128 workgroups with an f32 input, RMSNorm aside:
    //  eight wavefronts quantising one block each, the six past the groups
    //  skipping the walk -- with SmolLM-135M's w2, 36 workgroups, its decode
    //  measured 1.4 % more tokens/s; at 352 and 256 workgroups (5632 x 2048,
    //  2048 x 2048) the eight were 0.5-1 us slower.  RMSNorm keeps two, as the
    //  two-weight launch does, so that the two give the same sums)
    if (ng <= 8 && fused && p.xf != RL_XF_NORM && grid <= 128)
        return launch_g<TYPE, RG_ROWS, 8, 1, NPG, true, false, true>(p, grid, fused, dump, s);
    if (ng <= 8) return launch_g<TYPE, RG_ROWS, 2, 1, NPG, true>(p, grid, fused, dump, s);
    if (ng <= 16) return launch_g<TYPE, RG_ROWS, 4, 1, NPG, true>(p, grid, fused, dump, s);
    if (ng <= 32) return launch_g<TYPE, RG_ROWS, 8, 1, NPG, true>(p, grid, fused, dump, s);
    if constexpr (Q80) return hipErrorNotSupported;  // Q8_0: up to 32 groups
    else {  // as many wavefronts as the groups need (four each): none only waits
        constexpr int PW = Q6 || NPG == 11 ? 7 : 6;
        if (ng <= 48) return launch_g<TYPE, RG_ROWS, 12, 1, PW, false>(p, grid, fused, dump, s);
        if (ng <= 56) return launch_g<TYPE, RG_ROWS, 14, 1, PW, false>(p, grid, fused, dump, s);
        return launch_g<TYPE, RG_ROWS, 16, 1, PW, false>(p, grid, fused, dump, s);
    }
}

}  // namespace

bool rowlane_matvec_applies(int type, int64_t n, int64_t k) {
    // Q8_0: rows of whole 256-element groups, up to 32 of them
    const int64_t maxg = type == TYPE_Q8_0 ? 32 : RL_MAXG;
    return (type == TYPE_Q4_K || type == TYPE_Q5_K || type == TYPE_Q6_K || type == TYPE_Q8_0 || type == TYPE_Q4_0 ||
            type == TYPE_Q5_0 || type == TYPE_Q2_K || type == TYPE_Q3_K) && k % QK_K == 0 && k > 0 &&
           k / QK_K <= maxg && n <= 0x7fffffff && (rows56(type, n, (int)(k / QK_K)) || n >= RG_MIN_N);
}

bool rowlane_xf_applies(int type, int64_t n, int64_t k, int kind) {
    return rowlane_matvec_applies(type, n, k) && (kind != RL_XF_NORM || k / QK_K <= RL_NORM_MAXG);
}

namespace {
// RlParams of one weight (checks shared by both entry points)
hipError_t rl_params(const WLayout &w, int64_t n, int64_t k, const float *x, const ActPlanes *act, float *y,
                     int32_t *S, int32_t *Smin, const RlXf *xf, RlParams &p) {
    if (!rowlane_matvec_applies(w.type, n, k)) return hipErrorNotSupported;
    if (!w.slab || !y || (!x && !act) || (S == nullptr) != (Smin == nullptr)) return hipErrorInvalidValue;
    if (xf && (!x || S || (xf->kind != RL_XF_NORM && xf->kind != RL_XF_SILU) || (xf->kind == RL_XF_NORM && !xf->w)))
        return hipErrorInvalidValue;
    if (xf && !rowlane_xf_applies(w.type, n, k, xf->kind)) return hipErrorNotSupported;
    if (xf && xf->swiglu && n % RB) return hipErrorInvalidValue;  // whole 8-row blocks of four gate, four up rows
    if (xf && xf->swiglu && xf->amax) return hipErrorInvalidValue;
    const int ng = (int)(k / QK_K);
    const int npg = slabs_of(w.type);
    if (w.ng != ng || w.rb_stride != (int64_t)ng * npg * 128) return hipErrorInvalidValue;
    if ((w.type == TYPE_Q6_K || w.type == TYPE_Q2_K) && !w.d) return hipErrorInvalidValue;
    if (x && ((uintptr_t)x & 15)) return hipErrorInvalidValue;
    const bool wide = rows56(w.type, n, ng);
    if ((int64_t)(wide ? RL_ROWS : RG_ROWS) / RB * w.rb_stride >= ((int64_t)1 << 31)) return hipErrorNotSupported;
    p.w = w.slab;
    p.wd = w.d;
    p.rb_stride = w.rb_stride;
    p.n = (int)n;
    p.k = (int)k;
    p.ng = ng;
    p.x = x;
    p.xf = xf ? xf->kind : RL_XF_NONE;
    p.xdelta = xf ? xf->delta : nullptr;
    p.xnorm = xf ? xf->w : nullptr;
    p.xout = xf ? xf->xout : nullptr;
    p.eps = xf ? xf->eps : 0.0f;
    p.act = act ? *act : ActPlanes{};
    p.y = y;
    p.swiglu = xf && xf->swiglu ? 1 : 0;
    p.amax = xf ? xf->amax : nullptr;
    p.S = S;
    p.Smin = Smin;
    return hipSuccess;
}

template <int T1, int T2, int R, int W, bool WQ>
hipError_t launch_two_rl(const RlParams &p1, const RlParams &p2, int g1, int g2, int kind, hipStream_t s) {
    if (!rl::grid_ok(R, p1.n, g1, false) || !rl::grid_ok(R, p2.n, g2, false)) return hipErrorInvalidValue;
    if (WQ && p1.ng > W) return hipErrorInvalidValue;  // a wavefront for every block
    if (kind == RL_XF_NORM) rl2_kernel<T1, T2, R, W, RL_XF_NORM, WQ><<<g1 + g2, W * 64, 0, s>>>(p1, p2, g1);
    else if (kind == RL_XF_SILU) rl2_kernel<T1, T2, R, W, RL_XF_SILU, WQ><<<g1 + g2, W * 64, 0, s>>>(p1, p2, g1);
    else rl2_kernel<T1, T2, R, W, RL_XF_NONE, WQ><<<g1 + g2, W * 64, 0, s>>>(p1, p2, g1);
    return hipGetLastError();
}

template <int R, int W, bool WQ = false>
hipError_t launch_two_w(const RlParams &p1, const RlParams &p2, int t1, int t2, int kind, hipStream_t s) {
    const int g1 = (p1.n + R - 1) / R, g2 = (p2.n + R - 1) / R;
    if (t1 == TYPE_Q4_K && t2 == TYPE_Q6_K) return launch_two_rl<TYPE_Q4_K, TYPE_Q6_K, R, W, WQ>(p1, p2, g1, g2, kind, s);
    if (t1 == TYPE_Q4_K && t2 == TYPE_Q4_K) return launch_two_rl<TYPE_Q4_K, TYPE_Q4_K, R, W, WQ>(p1, p2, g1, g2, kind, s);
    if (t1 == TYPE_Q6_K && t2 == TYPE_Q4_K) return launch_two_rl<TYPE_Q6_K, TYPE_Q4_K, R, W, WQ>(p1, p2, g1, g2, kind, s);
    return launch_two_rl<TYPE_Q6_K, TYPE_Q6_K, R, W, WQ>(p1, p2, g1, g2, kind, s);
}
}  // namespace

hipError_t launch_rowlane_matvec(const WLayout &w, int64_t n, int64_t k, const float *x, const ActPlanes *act,
                                 float *y, int32_t *S, int32_t *Smin, hipStream_t s, const RlXf *xf) {
    RlParams p;
    const hipError_t e = rl_params(w, n, k, x, act, y, S, Smin, xf, p);
    if (e != hipSuccess) return e;
    const bool wide = rows56(w.type, n, p.ng), fused = x != nullptr, dump = S != nullptr;
    if (w.type == TYPE_Q6_K) return launch_type<TYPE_Q6_K>(p, n, p.ng, wide, fused, dump, s);
    if (w.type == TYPE_Q8_0) return launch_type<TYPE_Q8_0>(p, n, p.ng, wide, fused, dump, s);
    if (w.type == TYPE_Q5_K) return launch_type<TYPE_Q5_K>(p, n, p.ng, wide, fused, dump, s);
    if (w.type == TYPE_Q4_0) return launch_type<TYPE_Q4_0>(p, n, p.ng, wide, fused, dump, s);
    if (w.type == TYPE_Q5_0) return launch_type<TYPE_Q5_0>(p, n, p.ng, wide, fused, dump, s);
    if (w.type == TYPE_Q2_K) return launch_type<TYPE_Q2_K>(p, n, p.ng, wide, fused, dump, s);
    if (w.type == TYPE_Q3_K) return launch_type<TYPE_Q3_K>(p, n, p.ng, wide, fused, dump, s);
    return launch_type<TYPE_Q4_K>(p, n, p.ng, wide, fused, dump, s);
}

hipError_t launch_rowlane_matvec2(const WLayout &w1, int64_t n1, float *y1, const WLayout &w2, int64_t n2, float *y2,
                                  int64_t k, const float *x, const RlXf &xf, hipStream_t s) {
    if (xf.swiglu || xf.amax) return hipErrorNotSupported;
    RlParams p1, p2;
    hipError_t e = rl_params(w1, n1, k, x, nullptr, y1, nullptr, nullptr, &xf, p1);
    if (e != hipSuccess) return e;
    RlXf xf2 = xf;
    xf2.xout = nullptr;  // the residual is written once, by the first weight's workgroup 0
    if ((e = rl_params(w2, n2, k, x, nullptr, y2, nullptr, nullptr, &xf2, p2)) != hipSuccess) return e;
    const int ng = p1.ng;
    auto kq = [](int t) { return t == TYPE_Q4_K || t == TYPE_Q6_K; };
    if (!kq(w1.type) || !kq(w2.type)) return hipErrorNotSupported;
    if (rows56(w1.type, n1, ng) || rows56(w2.type, n2, ng)) return hipErrorNotSupported;  // 16- and 8-row forms only
    if (ng > 32) return hipErrorNotSupported;  // four or eight wavefronts
    // both weights in the form a launch of their own takes, so that the sums
    // are the same
    const bool e1 = rows8(n1, ng), e2 = rows8(n2, ng);
    if (e1 != e2) return hipErrorNotSupported;
    if (e1) return ng <= 16 ? launch_two_w<RE_ROWS, 4>(p1, p2, w1.type, w2.type, xf.kind, s)
                            : launch_two_w<RE_ROWS, 8>(p1, p2, w1.type, w2.type, xf.kind, s);
    // (as the single launches: two wavefronts from 8 groups down, so that no
    //  wavefront only quantises and waits)
    return ng <= 8    ? launch_two_w<RG_ROWS, 2>(p1, p2, w1.type, w2.type, xf.kind, s)
           : ng <= 16 ? launch_two_w<RG_ROWS, 4>(p1, p2, w1.type, w2.type, xf.kind, s)
                      : launch_two_w<RG_ROWS, 8>(p1, p2, w1.type, w2.type, xf.kind, s);
}

}  // namespace aq
