// k_attn.hip -- Llama attention over the KV cache on gfx950: the decode step
// (one query position, the context split over workgroups) and the prompt
// (prefill: every position of the prompt, causal).  Both follow
// candle-transformers 0.8.4 quantized_llama's attention, which
// native/arm_ai_nif/src/llama_candle.rs:93 (prompt at offset 0) and :119 (one
// token at offset `offset`) run:
//   q, k = rope_i(q), rope_i(k) at their positions (interleaved pairs
//   (2i, 2i+1) rotated by pos * theta_i, from cos/sin tables [max_seq][hd/2]);
//   k, v appended to the cache [n_kv][max_seq][hd] at their positions;
//   each query head h attends with kv head h / (n_head / n_kv);
//   softmax over (q . k_p) / sqrt(hd) with the causal mask p > position
//   (candle masks whenever more than one position is fed), then . v.
// f32 throughout (no fast-math, no FMA contraction of the rotation); sums are
// reordered relative to candle's loops, so results agree within rounding.
#include "aq_internal.h"

namespace aq {

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

// Sum / max over aligned groups of N = 16 or 32 lanes; every lane of a group
// gets the result (DPP within 16-lane rows, one cross-row swap for 32).
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(N == 16 || N == 32, "16- or 32-lane groups");
    v += dpp_f<DPP_QUAD_XOR1>(v);
    v += dpp_f<DPP_QUAD_XOR2>(v);
    v += dpp_f<DPP_HALF_MIRROR>(v);
    v += dpp_f<DPP_ROW_MIRROR>(v);
    if (N == 32) v += __shfl_xor(v, 16);
    return v;
}
__device__ __forceinline__ float group16_max(float v) {
    v = fmaxf(v, dpp_f<DPP_QUAD_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_QUAD_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_MIRROR>(v));
    return v;
}
__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float dot4(const float4 a, const float4 b) {
    return __builtin_fmaf(a.x, b.x, __builtin_fmaf(a.y, b.y, __builtin_fmaf(a.z, b.z, a.w * b.w)));
}
__device__ __forceinline__ void axpy4(float4 &acc, float w, const float4 x) {
    acc.x = __builtin_fmaf(w, x.x, acc.x);
    acc.y = __builtin_fmaf(w, x.y, acc.y);
    acc.z = __builtin_fmaf(w, x.z, acc.z);
    acc.w = __builtin_fmaf(w, x.w, acc.w);
}
constexpr float4 ZERO4 = {0.0f, 0.0f, 0.0f, 0.0f};

// ------------------------------------------------------------------ decode
// Two launches.  attn_split_kernel: grid (slices, n_kv kv heads), 256
// threads, for the S slices of the workspace or, when max_seq is shorter,
// the ceil(max_seq / 16) that can ever hold positions.  Workgroup (s, g) takes the positions [s*len, (s+1)*len) of
// 0..pos (len = max(16, ceil((pos+1)/S))) for all REP = n_head / n_kv query
// heads of kv head g, so every cached k, v row is read once per step (the
// query heads of a group share it), and writes, per query head, the slice's
// max score m, the sum l of e^(score - m) and the unnormalised o = sum of
// e^(score - m) v to its partial record.  The workgroup whose slice holds pos
// rotates k, stores k and v at pos, and uses its LDS copy for that position;
// slices past the context exit.  attn_combine_kernel: one wavefront per query
// head, M = max m_s, out = sum e^(m_s - M) o_s / sum e^(m_s - M) l_s.  (A
// last-arriving-workgroup combine in the first launch measured slower here:
// its device-scope release and the counter atomics of 256 workgroups cost
// more than the second launch.)
constexpr int SPL_THREADS = 256;
constexpr int SPL_MIN_LEN = 16;     // positions per slice at least (slices of 16 measured faster than 32:
                                    // more, shorter workgroups on the latency-bound step)
constexpr int SPL_MAX_LEN = 256;    // positions per slice at most (LDS scores)
constexpr int SPL_MAX_SLICES = 256;
constexpr int SPL_MAX_REP = 8;

// The slices that can ever hold positions: len >= SPL_MIN_LEN, so ns <=
// ceil(max_seq / SPL_MIN_LEN) (and ns <= S) at every position.
__host__ __device__ __forceinline__ int split_max_slices(int S, int max_seq) {
    const int c = (max_seq + SPL_MIN_LEN - 1) / SPL_MIN_LEN;
    return c < S ? c : S;
}

// the slice length and the number of slices that hold positions, for n = pos + 1
__device__ __forceinline__ void split_shape(int n, int S, int &len, int &ns) {
    len = (n + S - 1) / S;
    if (len < SPL_MIN_LEN) len = SPL_MIN_LEN;
    ns = (n + len - 1) / len;
}

template <int HD4, int REP>
__global__ __launch_bounds__(SPL_THREADS) void attn_split_kernel(
    const float *__restrict__ qk, const float *__restrict__ v, const float *__restrict__ cosb,
    const float *__restrict__ sinb, const int64_t *__restrict__ d_pos, float *__restrict__ kc, float *__restrict__ vc,
    int n_head, int max_seq, int S, float *__restrict__ part) {
    constexpr int hd = 4 * HD4;
    constexpr int G = SPL_THREADS / HD4;             // position groups of the value pass
    constexpr int PSTR = REP * hd + 2 * SPL_MAX_REP; // floats per partial record: o[REP][hd], m[8], l[8]
    constexpr int RPI = 64 / HD4;                    // key rows per wave load
    constexpr int RPP = RPI * (SPL_THREADS / 64);    // key rows per workgroup pass
    constexpr int KU = SPL_MIN_LEN / RPP;            // key passes loaded at the start (a whole minimum slice)
    constexpr int VU = SPL_MIN_LEN / G;              // value rows per thread loaded at the start
    static_assert(KU >= 1 && KU * RPP == SPL_MIN_LEN && VU >= 1 && VU * G == SPL_MIN_LEN,
                  "a minimum slice is whole key passes and whole value rounds");
    __shared__ __align__(16) float qs[REP * hd];
    __shared__ __align__(16) float ks[hd];
    __shared__ __align__(16) float vs[hd];
    __shared__ float sc[REP * SPL_MAX_LEN];
    __shared__ float4 accs[G * REP * HD4];

    const int s = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int c = lane % HD4, d4 = tid % HD4, g = tid / HD4;
    float *kh = kc + (int64_t)kvh * max_seq * hd;
    float *vh = vc + (int64_t)kvh * max_seq * hd;

    // Loads whose addresses do not depend on pos go out together with the
    // position load: q's values, the new k's and v's, and -- when the S
    // slices of SPL_MIN_LEN cover max_seq, so that slice s is positions
    // [SPL_MIN_LEN s, SPL_MIN_LEN (s + 1)) at every pos -- the cached rows of
    // the slice's first SPL_MIN_LEN positions (those at or past pos are
    // zeroed once pos is known).  Otherwise those rows are loaded after it.
    constexpr int QN = (REP * hd / 2 + SPL_THREADS - 1) / SPL_THREADS;  // q pairs per thread
    static_assert(hd / 2 + hd <= SPL_THREADS, "one of the new k's pairs or v's values per thread");
    float qa[QN], qb[QN];
#pragma unroll
    for (int u = 0; u < QN; u++) {
        const int i = tid + u * SPL_THREADS, hh = i / (hd / 2), j = i % (hd / 2);
        const float *q0 = qk + (int64_t)(kvh * REP + hh) * hd;
        qa[u] = i < REP * hd / 2 ? q0[2 * j] : 0.0f;
        qb[u] = i < REP * hd / 2 ? q0[2 * j + 1] : 0.0f;
    }
    float na = 0.0f, nb = 0.0f;  // thread t < hd / 2: the new k's pair t; t < hd / 2 + hd: v's value t - hd / 2
    {
        const float *k0 = qk + (int64_t)n_head * hd + (int64_t)kvh * hd;
        if (tid < hd / 2) {
            na = k0[2 * tid];
            nb = k0[2 * tid + 1];
        } else if (tid < hd / 2 + hd) {
            na = v[(int64_t)kvh * hd + tid - hd / 2];
        }
    }
    const bool fixed = (int64_t)SPL_MIN_LEN * S >= max_seq;  // uniform
    float4 kv0[KU], vp[VU];
    if (fixed) {
        const int pf = s * SPL_MIN_LEN;
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int p = pf + u * RPP + wave * RPI + lane / HD4;
            kv0[u] = p < max_seq ? ((const float4 *)(kh + (int64_t)p * hd))[c] : ZERO4;
        }
#pragma unroll
        for (int u = 0; u < VU; u++) {
            const int p = pf + g + u * G;
            vp[u] = p < max_seq ? *(const float4 *)(vh + (int64_t)p * hd + 4 * d4) : ZERO4;
        }
    }

    const int pos = (int)*d_pos;
    if (pos < 0 || pos >= max_seq) return;  // the host checks; this never indexes out of the cache
    const int n = pos + 1;
    int len, ns;
    split_shape(n, S, len, ns);
    if (s >= ns) return;
    float *pw = part + ((int64_t)kvh * S + s) * PSTR;
    const int p0 = s * len, np = min(p0 + len, n) - p0;  // (fixed: len = SPL_MIN_LEN, p0 = pf)
    const bool has_pos = p0 + np == n;

    // the cached rows of the slice's first SPL_MIN_LEN positions (before pos
    // only): in flight while q and k rotate
#pragma unroll
    for (int u = 0; u < KU; u++) {
        const int i = u * RPP + wave * RPI + lane / HD4, p = p0 + i;
        if (!fixed) kv0[u] = i < np && p < pos ? ((const float4 *)(kh + (int64_t)p * hd))[c] : ZERO4;
        else if (!(i < np && p < pos)) kv0[u] = ZERO4;
    }
#pragma unroll
    for (int u = 0; u < VU; u++) {
        const int i = g + u * G, p = p0 + i;
        if (!fixed) vp[u] = i < np && p < pos ? *(const float4 *)(vh + (int64_t)p * hd + 4 * d4) : ZERO4;
        else if (!(i < np && p < pos)) vp[u] = ZERO4;
    }

    const float *cr = cosb + (int64_t)pos * (hd / 2), *sr = sinb + (int64_t)pos * (hd / 2);
#pragma unroll
    for (int u = 0; u < QN; u++) {
        const int i = tid + u * SPL_THREADS, hh = i / (hd / 2), j = i % (hd / 2);
        if (i < REP * hd / 2) {
            const float a = qa[u], b = qb[u], cc = cr[j], sn = sr[j];
            qs[hh * hd + 2 * j] = a * cc - b * sn;
            qs[hh * hd + 2 * j + 1] = a * sn + b * cc;
        }
    }
    if (has_pos) {  // k's hd / 2 rotated pairs, then v's hd values
        if (tid < hd / 2) {
            const float a = na, b = nb, cc = cr[tid], sn = sr[tid];
            ks[2 * tid] = a * cc - b * sn;
            ks[2 * tid + 1] = a * sn + b * cc;
        } else if (tid < hd / 2 + hd) {
            vs[tid - hd / 2] = na;
        }
    }
    __syncthreads();
    if (has_pos) {
        for (int t = tid; t < hd; t += SPL_THREADS) {
            kh[(int64_t)pos * hd + t] = ks[t];
            vh[(int64_t)pos * hd + t] = vs[t];
        }
#pragma unroll
        for (int u = 0; u < KU; u++)
            if (u * RPP + wave * RPI + lane / HD4 == np - 1) kv0[u] = ((const float4 *)ks)[c];
#pragma unroll
        for (int u = 0; u < VU; u++)
            if (g + u * G == np - 1) vp[u] = ((const float4 *)vs)[d4];
    }

    // scores: HD4 lanes per key row (lane c holds float4 c of each query
    // head), the row's REP dots summed over the lane group
    float4 qv[REP];
#pragma unroll
    for (int hh = 0; hh < REP; hh++) qv[hh] = ((const float4 *)(qs + hh * hd))[c];
    const float rs = sqrtf((float)hd);
    auto score_rows = [&](const float4 *kv, int b0, int nu) {
        for (int u = 0; u < nu; u++) {
            const int i = b0 + u * RPP + wave * RPI + lane / HD4;
#pragma unroll
            for (int hh = 0; hh < REP; hh++) {
                const float d = group_sum<HD4>(dot4(qv[hh], kv[u]));
                if (i < np && c == 0) sc[hh * SPL_MAX_LEN + i] = d / rs;
            }
        }
    };
    score_rows(kv0, 0, KU);
    for (int b0 = KU * RPP; b0 < np; b0 += KU * RPP) {  // slices longer than the minimum
        float4 kv[KU];
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int i = b0 + u * RPP + wave * RPI + lane / HD4, p = p0 + i;
            kv[u] = ZERO4;
            if (i < np) kv[u] = p < pos ? ((const float4 *)(kh + (int64_t)p * hd))[c] : ((const float4 *)ks)[c];
        }
        score_rows(kv, b0, KU);
    }
    __syncthreads();

    // per query head: the slice's max and e_p = exp(score - max), one wave per head
    for (int hh = wave; hh < REP; hh += SPL_THREADS / 64) {
        float mx = -INFINITY;
        for (int i = lane; i < np; i += 64) mx = fmaxf(mx, sc[hh * SPL_MAX_LEN + i]);
        mx = wave_max_f(mx);
        float sum = 0.0f;
        for (int i = lane; i < np; i += 64) {
            const float e = expf(sc[hh * SPL_MAX_LEN + i] - mx);
            sc[hh * SPL_MAX_LEN + i] = e;
            sum += e;
        }
        sum = wave_sum_f(sum);
        if (lane == 0) {
            pw[REP * hd + hh] = mx;
            pw[REP * hd + SPL_MAX_REP + hh] = sum;
        }
    }
    __syncthreads();

    // o[hh][d] = sum_p e_p v_p[d]: thread (d4, g) takes positions g (mod G)
    float4 acc[REP];
#pragma unroll
    for (int hh = 0; hh < REP; hh++) acc[hh] = ZERO4;
#pragma unroll
    for (int u = 0; u < VU; u++) {
        const int i = g + u * G;
        if (i < np) {
#pragma unroll
            for (int hh = 0; hh < REP; hh++) axpy4(acc[hh], sc[hh * SPL_MAX_LEN + i], vp[u]);
        }
    }
    for (int i0 = g + VU * G; i0 < np; i0 += 2 * G) {
        float4 v4[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int i = i0 + u * G, p = p0 + i;
            v4[u] = ZERO4;
            if (i < np) v4[u] = p < pos ? *(const float4 *)(vh + (int64_t)p * hd + 4 * d4) : ((const float4 *)vs)[d4];
        }
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int i = i0 + u * G;
            if (i < np) {
#pragma unroll
                for (int hh = 0; hh < REP; hh++) axpy4(acc[hh], sc[hh * SPL_MAX_LEN + i], v4[u]);
            }
        }
    }
#pragma unroll
    for (int hh = 0; hh < REP; hh++) accs[(g * REP + hh) * HD4 + d4] = acc[hh];
    __syncthreads();
    for (int f = tid; f < REP * HD4; f += SPL_THREADS) {
        float4 t = accs[f];
        for (int gg = 1; gg < G; gg++) {
            const float4 u4 = accs[gg * REP * HD4 + f];
            t.x += u4.x;
            t.y += u4.y;
            t.z += u4.z;
            t.w += u4.w;
        }
        ((float4 *)pw)[f] = t;  // f = hh * HD4 + d4
    }
}

// One wavefront per query head h (kv head h / REP, record slot h % REP).
// Every lane loads its own output dims of the first CS slices and the m, l
// of slices lane, lane + 64, ... in one round trip, issued together with the
// position load: records sit at fixed places, so the loads do not wait for
// pos, and the records past the context (left by earlier calls) are masked
// out once pos gives the slice count ns.  M = max m_s, weights e^(m_s - M)
// through LDS; then each lane sums its hd / 64 dims over the slices.
template <int HD4, int REP>
__global__ __launch_bounds__(64) void attn_combine_kernel(const float *__restrict__ part, const int64_t *__restrict__ d_pos,
                                                         int max_seq, int S, float *__restrict__ out) {
    constexpr int hd = 4 * HD4;
    constexpr int DL = hd / 64;  // output dims per lane
    constexpr int PSTR = REP * hd + 2 * SPL_MAX_REP;
    constexpr int CS = 64 / DL;  // slices whose outputs are loaded up front
    constexpr int MU = SPL_MAX_SLICES / 64;  // m, l values per lane at most
    __shared__ float w[SPL_MAX_SLICES];
    const int h = blockIdx.x, kvh = h / REP, hh = h % REP, lane = threadIdx.x;
    const float *pk = part + (int64_t)kvh * S * PSTR;
    const int smax = split_max_slices(S, max_seq);  // no record past it is ever used
    float ov[CS][DL], mv[MU], lv[MU];
#pragma unroll
    for (int s2 = 0; s2 < CS; s2++)
#pragma unroll
        for (int e = 0; e < DL; e++) ov[s2][e] = s2 < smax ? pk[(int64_t)s2 * PSTR + hh * hd + lane + 64 * e] : 0.0f;
#pragma unroll
    for (int u = 0; u < MU; u++) {
        const int s2 = lane + 64 * u;
        mv[u] = s2 < smax ? pk[(int64_t)s2 * PSTR + REP * hd + hh] : 0.0f;
        lv[u] = s2 < smax ? pk[(int64_t)s2 * PSTR + REP * hd + SPL_MAX_REP + hh] : 0.0f;
    }
    const int pos = (int)*d_pos;
    if (pos < 0 || pos >= max_seq) return;
    int len, ns;
    split_shape(pos + 1, S, len, ns);
    float M = -INFINITY;
#pragma unroll
    for (int u = 0; u < MU; u++)
        if (lane + 64 * u < ns) M = fmaxf(M, mv[u]);
    M = wave_max_f(M);
    float L = 0.0f;
#pragma unroll
    for (int u = 0; u < MU; u++) {
        const int s2 = lane + 64 * u;
        if (s2 < ns) {
            const float e = expf(mv[u] - M);
            w[s2] = e;
            L = __builtin_fmaf(e, lv[u], L);
        }
    }
    L = wave_sum_f(L);
    __syncthreads();
    float o[DL];
#pragma unroll
    for (int e = 0; e < DL; e++) o[e] = 0.0f;
#pragma unroll
    for (int s2 = 0; s2 < CS; s2++)
        if (s2 < ns) {
#pragma unroll
            for (int e = 0; e < DL; e++) o[e] = __builtin_fmaf(w[s2], ov[s2][e], o[e]);
        }
    for (int s2 = CS; s2 < ns; s2++) {
#pragma unroll
        for (int e = 0; e < DL; e++) o[e] = __builtin_fmaf(w[s2], pk[(int64_t)s2 * PSTR + hh * hd + lane + 64 * e], o[e]);
    }
#pragma unroll
    for (int e = 0; e < DL; e++) out[(int64_t)h * hd + lane + 64 * e] = o[e] / L;
}

// ------------------------------------------------------------------ prefill
// 1) rope_kv_kernel: row i of the prompt (position index_pos + i): rotate its
//    k heads and store them, and its v heads, in the cache.  One workgroup
//    per row.
__global__ __launch_bounds__(256) void rope_kv_kernel(const float *__restrict__ k, int64_t ldk,
                                                      const float *__restrict__ v, int64_t ldv,
                                                      const float *__restrict__ cosb, const float *__restrict__ sinb,
                                                      int index_pos, int n_kv, int hd, int max_seq,
                                                      float *__restrict__ kc, float *__restrict__ vc) {
    const int i = blockIdx.x, p = index_pos + i, h2 = hd / 2;
    const float *kr = k + (int64_t)i * ldk, *vr = v + (int64_t)i * ldv;
    const float *cr = cosb + (int64_t)p * h2, *sr = sinb + (int64_t)p * h2;
    for (int j = threadIdx.x; j < n_kv * h2; j += 256) {
        const int g = j / h2, jj = j % h2;
        const float a = kr[g * hd + 2 * jj], b = kr[g * hd + 2 * jj + 1], c = cr[jj], sn = sr[jj];
        float *dst = kc + ((int64_t)g * max_seq + p) * hd + 2 * jj;
        dst[0] = a * c - b * sn;
        dst[1] = a * sn + b * c;
    }
    for (int j = threadIdx.x; j < n_kv * hd; j += 256) {
        const int g = j / hd, d = j % hd;
        vc[((int64_t)g * max_seq + p) * hd + d] = vr[j];
    }
}

// 2) attn_prefill_kernel: one workgroup of four wavefronts per (query tile
//    of 32 rows, query head), on the f32 matrix cores
//    (v_mfma_f32_32x32x2f32: f32 products, f32 sums).  Wavefront w takes the
//    key blocks w, w + 4, ... (32 cached positions each) up to the tile's
//    last position, and keeps a running max, sum and output per query row;
//    the four are combined through LDS at the end (M = max m_w, out = sum
//    e^(m_w - M) o_w / sum e^(m_w - M) l_w).
//    Scores are formed transposed, S^T[key][query] = K . Q^T: lane (j, hh)
//    holds query j against 16 keys, so the softmax of a query row needs only
//    its own registers and the other lane half (lane ^ 32).  Those registers
//    are also the B operand of the P . V product, taken as
//    O^T[dim][query] += V^T[dim][key] . P^T[key][query], so the output rows
//    stay with their lanes and no probability moves between lanes.  The head
//    dims of the score product are split between the lane halves (hh * hd/2
//    ..), so each lane reads its q and k rows as contiguous halves.
//    A block's V values are loaded before its score MFMAs and the next
//    block's K half-rows before its P . V MFMAs, so each load waits under the
//    other half's matrix work.  Workgroups are dispatched with the tiles that
//    have the most keys first.
//    The softmax runs in base 2: scores are scaled by log2(e) / sqrt(hd) once
//    and exponentiated by the hardware exp2 (v_exp_f32), so the running max
//    and sum are those of e^(s / sqrt(hd)) in base-2 units.  The output is
//    unchanged up to rounding: the scale is one multiply instead of a
//    division, and v_exp_f32 is within about an ulp of expf's result (the
//    output stays within 1e-6 of the f64 attention; 10 % faster than expf,
//    whose range reduction is about ten VALU instructions a value).
constexpr int PM_QT = 32, PM_KB = 32, PM_W = 4;

template <int HD>
__global__ __launch_bounds__(64 * PM_W) void attn_prefill_kernel(const float *__restrict__ q, int64_t ldq,
                                                                 const float *__restrict__ cosb,
                                                                 const float *__restrict__ sinb,
                                                                 const float *__restrict__ kc,
                                                                 const float *__restrict__ vc, int index_pos, int m,
                                                                 int n_head, int n_kv, int max_seq,
                                                                 float *__restrict__ out) {
    constexpr int H2 = HD / 2;   // head dims per lane half: the score MFMAs' K steps
    constexpr int NB = HD / 32;  // 32-row blocks of the output's head dims
    __shared__ float sm_m[PM_W][PM_QT], sm_l[PM_W][PM_QT];
    __shared__ float sm_o[PM_W][PM_QT][32 + 1];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int j = lane & 31, hh = lane >> 5;
    const int ntq = (m + PM_QT - 1) / PM_QT;
    const int rank = blockIdx.x / n_head, h = blockIdx.x % n_head;
    const int tq = ntq - 1 - rank;  // the tiles with the most keys first
    const int qb = tq * PM_QT, rows = min(PM_QT, m - qb);
    const int kvh = h / (n_head / n_kv);
    const float *kh = kc + (int64_t)kvh * max_seq * HD;
    const float *vh = vc + (int64_t)kvh * max_seq * HD;
    const int kend = index_pos + qb + rows;  // keys 0 .. kend - 1
    const int nkb = (kend + PM_KB - 1) / PM_KB;
    const int qpos = index_pos + qb + j;

    // this lane's query fragment: dims hh * H2 .. of row qb + j, rotated at qpos
    float qv[H2];
#pragma unroll
    for (int i = 0; i < H2; i++) qv[i] = 0.0f;
    if (j < rows) {
        const float *qr = q + (int64_t)(qb + j) * ldq + (int64_t)h * HD + hh * H2;
        const float *cr = cosb + (int64_t)qpos * (HD / 2) + hh * (H2 / 2);
        const float *sr = sinb + (int64_t)qpos * (HD / 2) + hh * (H2 / 2);
#pragma unroll
        for (int i = 0; i < H2 / 2; i++) {
            const float a = qr[2 * i], b = qr[2 * i + 1], c = cr[i], sn = sr[i];
            qv[2 * i] = a * c - b * sn;
            qv[2 * i + 1] = a * sn + b * c;
        }
    }

    const float sc2 = 1.4426950408889634f / sqrtf((float)HD);  // log2(e) / sqrt(hd)
    float mrun = -INFINITY, lrun = 0.0f;
    v16f o[NB];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[b][r] = 0.0f;

    // loads: a key block's V rows are issued before its score MFMAs and the
    // next block's K rows before its PV MFMAs, so each load's latency passes
    // under the other half's matrix work.  Rows past kend are clamped to the
    // last valid row (their probabilities are zero; the values stay finite).
    float kv[H2], vv[NB][16];
    auto load_k = [&](int kb) {
        const int krow = min(kb * PM_KB + j, kend - 1);
        const float4 *kr4 = (const float4 *)(kh + (int64_t)krow * HD + hh * H2);
#pragma unroll
        for (int i = 0; i < H2 / 4; i++) {
            const float4 t = kr4[i];
            kv[4 * i] = t.x;
            kv[4 * i + 1] = t.y;
            kv[4 * i + 2] = t.z;
            kv[4 * i + 3] = t.w;
        }
    };
    if (w < nkb) load_k(w);
    for (int kb = w; kb < nkb; kb += PM_W) {
        const int k0 = kb * PM_KB;
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int st = 0; st < 16; st++) {
                const int key = min(k0 + 8 * (st >> 2) + 4 * hh + (st & 3), kend - 1);
                vv[b][st] = vh[(int64_t)key * HD + 32 * b + j];
            }
        // S^T[key][query] = sum over the head dims of K[key] * Q[query]
        v16f s, s1;  // two independent chains (even and odd steps), added at the end
#pragma unroll
        for (int r = 0; r < 16; r++) s[r] = s1[r] = 0.0f;
#pragma unroll
        for (int d = 0; d < H2; d += 2) {
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[d], qv[d], s, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[d + 1], qv[d + 1], s1, 0, 0, 0);
        }
        s += s1;
        if (kb + PM_W < nkb) load_k(kb + PM_W);
        // lane (j, hh) register r: query j, key k0 + 8 (r / 4) + 4 hh + r % 4
        float pv[16];
        float bm = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int key = k0 + 8 * (r >> 2) + 4 * hh + (r & 3);
            pv[r] = key > qpos ? -INFINITY : s[r] * sc2;
            bm = fmaxf(bm, pv[r]);
        }
        bm = fmaxf(bm, __shfl_xor(bm, 32));
        const float mnew = fmaxf(mrun, bm);
        const float msafe = mnew == -INFINITY ? 0.0f : mnew;  // a block wholly past this query
        const float scale = __builtin_amdgcn_exp2f(mrun - msafe);
        float ps = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            pv[r] = __builtin_amdgcn_exp2f(pv[r] - msafe);
            ps += pv[r];
        }
        ps += __shfl_xor(ps, 32);
        lrun = __builtin_fmaf(lrun, scale, ps);
        mrun = mnew;
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[b][r] *= scale;
        // O^T[head dim][query] += V^T[head dim][key] . P^T[key][query]
#pragma unroll
        for (int st = 0; st < 16; st++)
#pragma unroll
            for (int b = 0; b < NB; b++) o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[b][st], pv[st], o[b], 0, 0, 0);
    }

    // combine the four wavefronts' key ranges: M = max m_w, out = sum e^(m_w - M) o_w / sum e^(m_w - M) l_w
    if (hh == 0) {
        sm_m[w][j] = mrun;
        sm_l[w][j] = lrun;
    }
    // 32-dim rounds: the threads split the tile's 32 rows x 32 dims
    constexpr int TPR = 2 * PM_W;       // threads per query row
    constexpr int DPT = 32 / TPR;       // dims per thread per round (8 or 4)
    const int qq = tid / TPR, part = tid % TPR;
#pragma unroll
    for (int b = 0; b < NB; b++) {
        __syncthreads();  // the previous round's reads are done (and m, l written)
#pragma unroll
        for (int r = 0; r < 16; r++) sm_o[w][j][8 * (r >> 2) + 4 * hh + (r & 3)] = o[b][r];
        __syncthreads();
        float ew[PM_W], M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < PM_W; ww++) M = fmaxf(M, sm_m[ww][qq]);
        const float Ms = M == -INFINITY ? 0.0f : M;
        float L = 0.0f;
#pragma unroll
        for (int ww = 0; ww < PM_W; ww++) {
            ew[ww] = __builtin_amdgcn_exp2f(sm_m[ww][qq] - Ms);
            L = __builtin_fmaf(ew[ww], sm_l[ww][qq], L);
        }
        if (qq < rows) {
            float res[DPT];
#pragma unroll
            for (int dd = 0; dd < DPT; dd++) {
                float acc = 0.0f;
#pragma unroll
                for (int ww = 0; ww < PM_W; ww++) acc = __builtin_fmaf(ew[ww], sm_o[ww][qq][part * DPT + dd], acc);
                res[dd] = acc / L;
            }
            float *orow = out + (int64_t)(qb + qq) * n_head * HD + (int64_t)h * HD + 32 * b + part * DPT;
            if constexpr (DPT % 4 == 0) {
#pragma unroll
                for (int u = 0; u < DPT / 4; u++)
                    ((float4 *)orow)[u] = make_float4(res[4 * u], res[4 * u + 1], res[4 * u + 2], res[4 * u + 3]);
            } else {
#pragma unroll
                for (int u = 0; u < DPT / 2; u++) ((float2 *)orow)[u] = make_float2(res[2 * u], res[2 * u + 1]);
            }
        }
    }
}

template <int HD4, int REP>
void launch_split(dim3 grid, const float *qk, const float *v, const float *cosb, const float *sinb,
                  const int64_t *d_pos, float *kc, float *vc, int n_head, int max_seq, int S, float *part, float *out,
                  hipStream_t s) {
    attn_split_kernel<HD4, REP><<<grid, SPL_THREADS, 0, s>>>(qk, v, cosb, sinb, d_pos, kc, vc, n_head, max_seq, S,
                                                            part);
    attn_combine_kernel<HD4, REP><<<(unsigned)n_head, 64, 0, s>>>(part, d_pos, max_seq, S, out);
}

}  // namespace

int attn_split_slices(int64_t n_kv, int64_t max_seq) {
    int64_t S = 256 / n_kv;
    if (S < 32) S = 32;
    while (S * SPL_MAX_LEN < max_seq) S *= 2;
    return S > SPL_MAX_SLICES ? 0 : (int)S;
}

size_t attn_split_workspace_bytes(int64_t n_head, int64_t n_kv, int64_t hd, int64_t max_seq) {
    const int S = attn_split_slices(n_kv, max_seq);
    if (S == 0) return (size_t)-1;
    const int64_t rep = n_head / n_kv;
    return (size_t)(n_kv * S) * (size_t)(rep * hd + 2 * SPL_MAX_REP) * 4;
}

hipError_t launch_attn_split(const float *qk, const float *v, const float *cosb, const float *sinb,
                             const int64_t *d_pos, float *kc, float *vc, int64_t n_head, int64_t n_kv, int64_t hd,
                             int64_t max_seq, float *out, float *part, size_t part_bytes, hipStream_t s) {
    if (n_head <= 0 || n_kv <= 0 || n_head % n_kv || n_kv > 65535) return hipErrorNotSupported;
    const int64_t rep = n_head / n_kv;
    if ((hd != 64 && hd != 128) || (rep != 1 && rep != 2 && rep != 3 && rep != 4 && rep != 8)) return hipErrorNotSupported;
    const int S = attn_split_slices(n_kv, max_seq);
    if (S == 0 || attn_split_workspace_bytes(n_head, n_kv, hd, max_seq) > part_bytes) return hipErrorNotSupported;
    // slices past split_max_slices never hold a position: no workgroup for them
    const dim3 grid((unsigned)split_max_slices(S, (int)max_seq), (unsigned)n_kv);
    const int nh = (int)n_head, ms = (int)max_seq;
#define AQ_SPLIT(H4, R) launch_split<H4, R>(grid, qk, v, cosb, sinb, d_pos, kc, vc, nh, ms, S, part, out, s)
    if (hd == 64) {
        switch (rep) {
        case 1: AQ_SPLIT(16, 1); break;
        case 2: AQ_SPLIT(16, 2); break;
        case 3: AQ_SPLIT(16, 3); break;
        case 4: AQ_SPLIT(16, 4); break;
        default: AQ_SPLIT(16, 8); break;
        }
    } else {
        switch (rep) {
        case 1: AQ_SPLIT(32, 1); break;
        case 2: AQ_SPLIT(32, 2); break;
        case 3: AQ_SPLIT(32, 3); break;
        case 4: AQ_SPLIT(32, 4); break;
        default: AQ_SPLIT(32, 8); break;
        }
    }
#undef AQ_SPLIT
    return hipGetLastError();
}

hipError_t launch_attn_prefill(const float *q, int64_t ldq, const float *k, int64_t ldk, const float *v, int64_t ldv,
                               const float *cosb, const float *sinb, int64_t index_pos, int64_t m, float *kc,
                               float *vc, int64_t n_head, int64_t n_kv, int64_t hd, int64_t max_seq, float *out,
                               hipStream_t s) {
    if (!q || !k || !v || !cosb || !sinb || !kc || !vc || !out) return hipErrorInvalidValue;
    if (m <= 0 || index_pos < 0 || max_seq <= 0 || index_pos + m > max_seq || max_seq > 0x7fffffff ||
        n_head <= 0 || n_kv <= 0 || n_head % n_kv || n_head > 65535)
        return hipErrorInvalidValue;
    if (hd != 64 && hd != 128) return hipErrorNotSupported;
    if (ldq < n_head * hd || ldk < n_kv * hd || ldv < n_kv * hd) return hipErrorInvalidValue;
    if (((uintptr_t)kc | (uintptr_t)vc | (uintptr_t)out) & 15) return hipErrorInvalidValue;
    rope_kv_kernel<<<(unsigned)m, 256, 0, s>>>(k, ldk, v, ldv, cosb, sinb, (int)index_pos, (int)n_kv, (int)hd,
                                               (int)max_seq, kc, vc);
    const unsigned grid = (unsigned)(((m + PM_QT - 1) / PM_QT) * n_head);
    if (hd == 64)
        attn_prefill_kernel<64><<<grid, 64 * PM_W, 0, s>>>(q, ldq, cosb, sinb, kc, vc, (int)index_pos, (int)m, (int)n_head,
                                                     (int)n_kv, (int)max_seq, out);
    else
        attn_prefill_kernel<128><<<grid, 64 * PM_W, 0, s>>>(q, ldq, cosb, sinb, kc, vc, (int)index_pos, (int)m,
                                                      (int)n_head, (int)n_kv, (int)max_seq, out);
    return hipGetLastError();
}

}  // namespace aq
