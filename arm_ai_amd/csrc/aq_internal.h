// aq_internal.h -- device layouts and helpers shared by the gfx950 kernels
// of libarm_ai_amd.so.  Not part of the public ABI (include/aq.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace aq {

constexpr int QK_K = 256;
constexpr int QK8_0 = 32;
constexpr int TYPE_Q4_0 = 2;
constexpr int TYPE_Q5_0 = 6;
constexpr int TYPE_Q8_0 = 8;
constexpr int TYPE_Q2_K = 10;
constexpr int TYPE_Q3_K = 11;
constexpr int TYPE_Q4_K = 12;
constexpr int TYPE_Q5_K = 13;
constexpr int TYPE_Q6_K = 14;
constexpr int TYPE_Q8_K = 15;

// ---------------------------------------------------------------------------
// Weight layout in HBM ("row-block tiles").  A weight row is cut into groups
// of 256 elements: one super-block for Q4_K / Q6_K, eight 32-element blocks
// for Q8_0.  Each group is a fixed number of 16-byte pieces (the repack at
// upload is lossless; same bytes, moved):
//   Q4_K (9 pieces = 144 B):  piece 0 = d f16, dmin f16, scales[12];
//                             pieces 1..8 = qs[0..127] in GGUF order.
//   Q5_K (11 pieces = 176 B): the GGUF block in order: piece 0 as Q4_K,
//                             pieces 1..2 = qh[0..31], 3..10 = qs[0..127].
//   Q6_K (13 pieces = 208 B + d plane): pieces 0..7 = ql[0..127],
//                             8..11 = qh[0..63], 12 = scales[16]; the f16 d of
//                             each super-block goes to a separate plane.
//   Q8_0 (17 pieces = 272 B): pieces 2j, 2j+1 = qs of block 8g+j, piece 16 =
//                             the eight f16 d; a row whose block count is not a
//                             multiple of 8 is padded with zero blocks.
//   Q4_0 (9 pieces = 144 B):  piece j = the 16 qs bytes of block 8g+j, piece 8
//                             = the eight f16 d; padded like Q8_0.
//   Q5_0 (11 pieces = 176 B): piece j = the 16 qs bytes of block 8g+j, pieces
//                             8 + j/4 bytes 4(j%4).. = its 32-bit qh, piece 10
//                             = the eight f16 d; padded like Q8_0.
//   Q2_K (5 pieces = 80 B + d plane): piece 0 = scales[16], 1..4 = qs[0..63];
//                             d and dmin (f16 each) go to a plane of 32-bit
//                             entries, d in the low half.
//   Q3_K (7 pieces = 112 B):  the GGUF block in order: pieces 0..1 = hmask,
//                             2..5 = qs, 6 = scales[12] then f16 d (2 bytes
//                             of padding).
// Rows are taken in blocks of 8 (the row count is padded with zero rows to a
// multiple of 8), and for each (row block, group, piece) the 8 rows' pieces
// are one 128-byte line:
//   byte offset of piece p of group g of row r =
//       (r/8) * rb_stride + (g * PIECES + p) * 128 + (r%8) * 16,
//   rb_stride = groups * PIECES * 128;
//   Q6_K d of (r, g): element ((r/8) * groups + g) * 8 + r%8 of the d plane
//   (16-bit entries; Q2_K: 32-bit entries at the same index).
// The decode matvec reads a tile with lanes (group, row) of an 8 x 8 block of
// a row block: eight full lines per load instruction.  The prefill GEMM reads
// it with lanes over 32 consecutive rows (output columns) of one group: four
// full lines per half-wavefront.
// ---------------------------------------------------------------------------
constexpr int RB = 8;  // rows per row block
struct WLayout {
    const uint8_t *slab = nullptr;  // row-block tiles
    const uint16_t *d = nullptr;    // Q6_K: [n/8][groups][8] f16; Q2_K: [n/8][groups][8] (f16 d, f16 dmin)
    int type = 0;
    int ng = 0;                     // groups per row
    int64_t rb_stride = 0;          // bytes per row block
};

__host__ __device__ constexpr int slabs_of(int type) {
    return type == TYPE_Q4_K ? 9 : type == TYPE_Q5_K ? 11 : type == TYPE_Q6_K ? 13 : type == TYPE_Q8_0 ? 17
         : type == TYPE_Q4_0 ? 9 : type == TYPE_Q2_K ? 5 : type == TYPE_Q3_K ? 7 : type == TYPE_Q5_0 ? 11 : 0;
}
// Weights whose activation is quantised to Q8_0 blocks of 32 (candle's
// VecDotType): Q8_0, Q4_0 and Q5_0.  The others use Q8_K.
__host__ __device__ constexpr bool act_q80(int type) { return type == TYPE_Q8_0 || type == TYPE_Q4_0 || type == TYPE_Q5_0; }
inline int groups_of(int type, int64_t k) {
    return act_q80(type) ? (int)((k / QK8_0 + 7) / 8) : (int)(k / QK_K);
}

// Quantised activation planes (written by the quantizer kernels):
//   qs    [m][k]      i8
//   d     [m][k/256]  f32 (Q8_K) or [m][k/32] f32 value of the f16 d (Q8_0)
//   d16   [m][k/32]   f16 bits of the Q8_0 d
//   bsums [m][k/16]   i16 (Q8_K)
//   bsum16 [m][k/16]  the same bsums as f16 bits (exact: |bsum| <= 2048), the
//                     A operand of the GEMM's f16 MFMA for the min term
//   q16   [m][k]      the qs as f16 bits, the activation operand of the
//                     f16-MFMA GEMMs (Q6_K, Q5_K); written by the Q8_K
//                     quantizers when the pointer is set (paths that feed no
//                     such GEMM clear it)
struct ActPlanes {
    int8_t *qs;
    float *d;
    uint16_t *d16;
    int16_t *bsums;
    uint16_t *bsum16;
    uint16_t *q16 = nullptr;
};

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Sizes of the activation planes for m rows of k (bytes, each plane 256-B aligned).
struct ActSizes {
    size_t qs, d, d16, bsums, bsum16, q16, total;
};
inline ActSizes act_sizes(int64_t m, int64_t k) {
    ActSizes s;
    s.qs = align_up((size_t)m * k, 256);
    s.d = align_up((size_t)m * (k / 32) * 4, 256);  // large enough for Q8_K (k/256) and Q8_0 (k/32)
    s.d16 = align_up((size_t)m * (k / 32) * 2, 256);
    s.bsums = align_up((size_t)m * (k / 16) * 2, 256);
    s.bsum16 = s.bsums;
    s.q16 = align_up((size_t)m * k * 2, 256);
    s.total = s.qs + s.d + s.d16 + s.bsums + s.bsum16 + s.q16;
    return s;
}
inline ActPlanes act_planes(void *base, int64_t m, int64_t k) {
    ActSizes s = act_sizes(m, k);
    uint8_t *p = (uint8_t *)base;
    ActPlanes a;
    a.qs = (int8_t *)p;
    a.d = (float *)(p + s.qs);
    a.d16 = (uint16_t *)(p + s.qs + s.d);
    a.bsums = (int16_t *)(p + s.qs + s.d + s.d16);
    a.bsum16 = (uint16_t *)(p + s.qs + s.d + s.d16 + s.bsums);
    a.q16 = (uint16_t *)(p + s.qs + s.d + s.d16 + s.bsums + s.bsum16);
    return a;
}

// ---------------------------------------------------------------------------
// Kernel launchers (defined in k_quantize.hip, k_matvec.hip, k_gemm.hip).
// Each checks the shapes its grid assumes and returns hipErrorInvalidValue
// rather than launching out of bounds.
// ---------------------------------------------------------------------------
hipError_t launch_quantize_q8k(const float *x, int64_t m, int64_t k, ActPlanes a, hipStream_t s);
hipError_t launch_quantize_q8_0(const float *x, int64_t m, int64_t k, ActPlanes a, hipStream_t s);
// GGUF blocks of n rows (device memory) -> those rows of the row-block tile
// layout.  dst_slab / dst_d point at the first destination row block (the
// first source row is a multiple of 8).  Padding (rows past n in the last row
// block, Q8_0 padding blocks) is not written: zero the tiles beforehand.
hipError_t launch_repack(int type, const uint8_t *src, int64_t n, int64_t k, uint8_t *dst_slab, uint16_t *dst_d,
                         hipStream_t s);
// GGUF Q4_0 / Q5_0 blocks of n rows -> those rows of a Q8_0 row-block tile
// layout holding the values (q - 8, q - 16) as int8 and the same f16 d (what
// the Q8_0 GEMM reads).  Padding is not written: zero the tiles beforehand.
hipError_t launch_expand_q80(int type, const uint8_t *src, int64_t n, int64_t k, uint8_t *dst_slab, hipStream_t s);
// Decode matvec (any m; batch rows are processed up to 8 at a time).  The
// activation is either f32 (x != nullptr: quantised inside the kernel,
// bit-identical to the quantizer kernels) or pre-quantised planes.
// S/Smin non-null selects the integer-dump variant ([m][n][blocks] int32).
hipError_t launch_matvec(const WLayout &w, int64_t n, int64_t k, const float *x, const ActPlanes *act, int64_t m,
                         float *y, int32_t *S, int32_t *Smin, hipStream_t s);
// Batch-1 matvec with one weight row per lane (k_rowlane.hip) for Q4_K,
// Q5_K, Q6_K, Q8_0, Q4_0, Q5_0, Q2_K and Q3_K weights of at least 256 rows, k
// a multiple of 256 and <= 16384 (8192 for Q8_0); hipErrorNotSupported for
// other shapes.  x (f32, quantised in the kernel) or act (pre-quantised
// planes of one row).  xf (x only, no dump): kind RL_XF_NORM quantises
// rms_norm(x + delta) * w (k <= 8192; workgroup 0 writes x + delta to
// xout), kind RL_XF_SILU takes x = [g | u] (2k floats) and quantises
// silu(g) * u.  swiglu (an output transform): the weight's rows are gate and
// up rows in pairs of four (swiglu_pair_rows: rows 8b..8b+3 gate rows
// 4b..4b+3, rows 8b+4..8b+7 the up rows of the same indices; n a multiple of
// 8), and y receives the n / 2 values silu(g) * u in place of the n sums.
constexpr int RL_XF_NONE = 0, RL_XF_NORM = 1, RL_XF_SILU = 2;
struct RlXf {
    int kind;  // RL_XF_NORM or RL_XF_SILU
    const float *delta, *w;
    float eps;
    float *xout;
    bool swiglu = false;
    // or null: per workgroup (grid: rowlane_grid), the bits of the largest
    // output and its row, the first of equal values (a NaN never wins)
    int2 *amax = nullptr;
};
int rowlane_grid(int type, int64_t n, int64_t k);
bool rowlane_matvec_applies(int type, int64_t n, int64_t k);
bool rowlane_xf_applies(int type, int64_t n, int64_t k, int kind);
hipError_t launch_rowlane_matvec(const WLayout &w, int64_t n, int64_t k, const float *x, const ActPlanes *act,
                                 float *y, int32_t *S, int32_t *Smin, hipStream_t s, const RlXf *xf = nullptr);
// Two weights of the same k on one f32 input and transform in one launch
// (both in the 16-row or both in the 8-row form, the one a launch of their
// own takes, so the sums are the same); hipErrorNotSupported otherwise.
hipError_t launch_rowlane_matvec2(const WLayout &w1, int64_t n1, float *y1, const WLayout &w2, int64_t n2, float *y2,
                                  int64_t k, const float *x, const RlXf &xf, hipStream_t s);
// Matvec of pre-quantised (Q8_K) rows on the int8 matrix cores, 8 rows per
// launch, Q4_K / Q6_K weights, k <= mmv_max_k().  Returns hipErrorNotSupported
// for other types and shapes (the caller then uses launch_matvec).  Shapes
// whose K is split over workgroups sum the parts in ws
// (mmv_workspace_bytes(type, n, k) bytes, 0 when there is no split).
int mmv_max_k();
size_t mmv_workspace_bytes(int type, int64_t n, int64_t k);
hipError_t launch_mmv(const WLayout &w, int64_t n, int64_t k, const ActPlanes &act, int64_t m, float *y, int32_t *S,
                      int32_t *Smin, void *ws, size_t ws_bytes, hipStream_t s);
// Prefill GEMM on MFMA (m > 8).  Returns hipErrorNotSupported for shapes it
// does not take; the caller then uses launch_matvec.  ws: gemm_workspace_bytes
// of scratch (split-K partials, summed by a second launch on the stream).
constexpr int GEMM_MAX_TILES = 1 << 20;
hipError_t launch_gemm(const WLayout &w, int64_t n, int64_t k, const ActPlanes &x, int64_t m, float *y, int32_t *S,
                       int32_t *Smin, void *ws, size_t ws_bytes, hipStream_t s);
// A Q4_K weight and a Q6_K / Q5_K weight of the same k on one activation
// (with its f16 quants plane) in one launch, the first unsplit, the second
// split over k as launch_gemm would (its partials in ws, gemm_workspace_bytes
// of the second weight's shape, and its reduce launch after).
// hipErrorNotSupported when the types differ from that, the rows need more
// than one launch, or the two together have more work items than the CUs
// hold at once (the caller then runs launch_gemm twice).
hipError_t launch_gemm_pair(const WLayout &w1, int64_t n1, float *y1, const WLayout &w2, int64_t n2, float *y2,
                            int64_t k, const ActPlanes &x, int64_t m, void *ws, size_t ws_bytes, hipStream_t s);
// Workspace bytes launch_gemm needs for this shape, or (size_t)-1 if the
// weight type / shape has no GEMM (the matvec then serves m > 8 too).
size_t gemm_workspace_bytes(int type, int64_t m, int64_t n, int64_t k);
// The Q6_K and Q5_K GEMM on f16 MFMA (k_gemm6.hip), reached through launch_gemm /
// gemm_workspace_bytes.  It reads the activation quants as f16 from
// ActPlanes::q16 when that is set (the quantizer wrote them), else converts
// them into its workspace first; the workspace also holds the split-K partials.
size_t gemm6_workspace_bytes(int64_t m, int64_t n, int64_t k);
hipError_t launch_gemm6(const WLayout &w, int64_t n, int64_t k, const ActPlanes &x, int64_t m, float *y, int32_t *S,
                        int32_t *Smin, void *ws, size_t ws_bytes, hipStream_t s);
// The Q8_0 GEMM on int8 MFMA (k_gemm8.hip), reached through launch_gemm /
// gemm_workspace_bytes; its workspace holds the split-K partial tiles.
size_t gemm8_workspace_bytes(int64_t m, int64_t n, int64_t k);
hipError_t launch_gemm8(const WLayout &w, int64_t n, int64_t k, const ActPlanes &x, int64_t m, float *y, int32_t *S,
                        int32_t *Smin, void *ws, size_t ws_bytes, hipStream_t s);
// Sums split-K partial tiles [tiles][splits][gbm][128] into y in split order.
hipError_t launch_splitk_reduce(const float *part, float *y, int m, int n, int ntm, int gbm, int splits, int tiles,
                                hipStream_t s);

// The NIF crate's own kernels (k_crate.hip; shape_ops.rs).
enum { CRATE_W_Q4_0 = 0, CRATE_W_I8 = 1, CRATE_W_F16 = 2 };
// out[i][j] = ((f32) sum_k a[i][k] w[j][k]) * (act_scales ? act_scales[i] : act_scale) * w_scales[j]
hipError_t launch_int8_matmul(const int8_t *a, const int8_t *w, const float *act_scales, float act_scale,
                              const float *w_scales, int64_t m, int64_t n, int64_t k, float *out, hipStream_t s);
hipError_t launch_quantize_int8_per_token(const float *a, int64_t m, int64_t k, int8_t *q, float *scales, hipStream_t s);
// f32 activations [m][k] x weights [n][k] (Q4_0-style, int8 or f16) -> [m][n]
hipError_t launch_weight_only_matmul(int wt, const float *a, const void *w, const float *w_scales, int64_t m, int64_t n,
                                     int64_t k, float *out, hipStream_t s);
// Q4_0 x Q8 GEMV; act: q4_x_q8_act_bytes(k) of scratch; q_out / s_out (optional)
// receive the quantised activation [k] i8 and its group scales [k/32].
size_t q4_x_q8_act_bytes(int64_t k);
hipError_t launch_q4_x_q8_gemv(const float *a, const uint8_t *w_packed, const float *w_scales, int64_t n, int64_t k,
                               float *out, void *act, int8_t *q_out, float *s_out, hipStream_t s);
hipError_t launch_quantize_int4_q4_0(const float *w, int64_t n, int64_t k, uint8_t *packed, float *scales, hipStream_t s);
hipError_t launch_dequantize_q6_k_crate(const uint8_t *blocks, int64_t nel, float *out, hipStream_t s);
hipError_t launch_dequant_rows(int wt, const void *table, const float *scales, int64_t ntab, const int64_t *rows,
                               int64_t nr, int64_t k, float *out, hipStream_t s);

// Decode matvec (m = 1, f32 input) with a fused input transform (k_matvec.hip):
// rms_norm(x + delta) * norm (workgroup 0 also writes x + delta to xout), or
// silu(g) * u with gu = [g (k) | u (k)].  hipErrorNotSupported when the row
// is too long for the fused norm (the caller then runs the two steps apart).
hipError_t launch_matvec_rmsnorm(const WLayout &w, int64_t n, int64_t k, const float *x, const float *delta,
                                 const float *norm, float eps, float *xout, float *y, hipStream_t s);
hipError_t launch_matvec_silu(const WLayout &w, int64_t n, int64_t k, const float *gu, float *y, hipStream_t s);
// The fused-norm matvec of a weight of gate and up rows in pairs of four
// (n a multiple of 8), writing the n / 2 values silu(g) * u to h; the
// row-per-lane forms only (hipErrorNotSupported otherwise).
hipError_t launch_matvec_rmsnorm_swiglu(const WLayout &w, int64_t n, int64_t k, const float *x, const float *delta,
                                        const float *norm, float eps, float *xout, float *h, hipStream_t s);
// The fused-norm matvec also leaving, per workgroup, its largest output and
// that row in amax (*nparts entries, at most max_parts); the row-per-lane
// forms only (hipErrorNotSupported otherwise).
hipError_t launch_matvec_rmsnorm_argmax(const WLayout &w, int64_t n, int64_t k, const float *x, const float *delta,
                                        const float *norm, float eps, float *y, int2 *amax, int max_parts,
                                        int *nparts, hipStream_t s);
// Two fused-norm matvecs of the same row in one launch (Q4_K / Q6_K weights
// w1 and w2, outputs y1 and y2); xout is written once.  hipErrorNotSupported
// for other types or rows too long to fuse.
hipError_t launch_matvec2_rmsnorm(const WLayout &w1, int64_t n1, float *y1, const WLayout &w2, int64_t n2, float *y2,
                                  int64_t k, const float *x, const float *delta, const float *norm, float eps,
                                  float *xout, hipStream_t s);

// Decode-step glue (k_decode.hip).
hipError_t launch_embed(const float *table, int64_t vocab, const int64_t *d_tok, int64_t m, int64_t hidden, float *out,
                        hipStream_t s);
hipError_t launch_rmsnorm(float *x, const float *delta, const float *w, int64_t m, int64_t n, float eps, float *out,
                          hipStream_t s);
hipError_t launch_silu_mul(const float *g, const float *u, int64_t ld, int64_t m, int64_t n, float *out, hipStream_t s);
// The prompt's norm and SwiGLU quantised to Q8_K in the same launch (the
// planes of a, q16 written when set): the values of launch_rmsnorm and
// launch_swiglu_pairs bit for bit (also written to out when it is non-null);
// n a multiple of 256.
hipError_t launch_rmsnorm_act(float *x, const float *delta, const float *w, int64_t m, int64_t n, float eps,
                              float *out, const ActPlanes &a, hipStream_t s);
hipError_t launch_swiglu_pairs_act(const float *y, int64_t ld, int64_t m, int64_t n, float *out, const ActPlanes &a,
                                   hipStream_t s);
// silu(g) * u of m rows of a paired gate|up weight's output (row stride ld,
// n = the number of pairs, a multiple of 4)
hipError_t launch_swiglu_pairs(const float *y, int64_t ld, int64_t m, int64_t n, float *out, hipStream_t s);
hipError_t launch_attn_decode(const float *qk, const float *v, const float *cosb, const float *sinb,
                              const int64_t *d_pos, float *kc, float *vc, int64_t n_head, int64_t n_kv, int64_t hd,
                              int64_t max_seq, float *out, hipStream_t s);
// k_attn.hip: the decode attention with the context split over workgroups
// and a second launch that combines the slices (hipErrorNotSupported for
// shapes it does not take: head_dim other than 64 or 128, more than 8 query
// heads per kv head, a workspace too small), its slice count and
// partial-record bytes, and the prompt's causal attention.
int attn_split_slices(int64_t n_kv, int64_t max_seq);
size_t attn_split_workspace_bytes(int64_t n_head, int64_t n_kv, int64_t hd, int64_t max_seq);
hipError_t launch_attn_split(const float *qk, const float *v, const float *cosb, const float *sinb,
                             const int64_t *d_pos, float *kc, float *vc, int64_t n_head, int64_t n_kv, int64_t hd,
                             int64_t max_seq, float *out, float *part, size_t part_bytes, hipStream_t s);
hipError_t launch_attn_prefill(const float *q, int64_t ldq, const float *k, int64_t ldk, const float *v, int64_t ldv,
                               const float *cosb, const float *sinb, int64_t index_pos, int64_t m, float *kc,
                               float *vc, int64_t n_head, int64_t n_kv, int64_t hd, int64_t max_seq, float *out,
                               hipStream_t s);
hipError_t launch_argmax(const float *x, int64_t n, int64_t *d_tok, int64_t *d_pos, int64_t *hist, int64_t hist_len,
                         hipStream_t s);
// The greedy pick from per-workgroup (value bits, row) pairs (the first row
// of the largest value), then that token's embedding row into xout.
// Per-workgroup first maxima of x (one (value bits, index) pair per 512
// values, at most max_parts) for launch_argmax_parts_embed.
hipError_t launch_argmax_parts(const float *x, int64_t n, int2 *parts, int max_parts, int *nparts, hipStream_t s);
hipError_t launch_argmax_parts_embed(const int2 *parts, int nparts, int64_t *d_tok, int64_t *d_pos, int64_t *hist,
                                     int64_t hist_len, const float *table, int64_t vocab, int64_t hidden, float *xout,
                                     hipStream_t s);

}  // namespace aq

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
#ifdef __HIPCC__
namespace aq {

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }
// Bits 0..3 of n (n < 16) to bit 4 of bytes 0..3: n * 0x204081 places bit i
// of n at bit 9i (no overlap; a 24-bit multiply).
__device__ __forceinline__ uint32_t spread4(uint32_t n) { return ((n * 0x204081u) & 0x01010101u) << 4; }

// Raw buffer accesses through a descriptor over [base, base + bytes): a lane
// whose offset lies past the range reads zeros / drops its store without a
// memory access, so the loads of a pipeline can be issued unconditionally
// (no branches around them, hence exact s_waitcnt counts).  BUF_OOB is an
// offset past every range (bytes < 2^31).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t BUF_OOB = 0x80000000u;
constexpr int BUF_NT = 2;  // cache policy: nontemporal (streamed once)
// Bit casts go through a by-value scalar: this clang's __builtin_bit_cast
// applied directly to an ext_vector element (v.y) reads element 0.
__device__ __forceinline__ float u32_as_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ uint32_t f32_as_u32(float f) { return __builtin_bit_cast(uint32_t, f); }
__device__ __forceinline__ rsrc_t buf_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// Raw buffer loads of 16 (4) bytes per lane straight into LDS: lane i's bytes
// land at lds + 16 * i (4 * i); lds must be wave-uniform.  (Kept in
// non-template functions: used directly inside a kernel template, this
// builtin stopped the host-side launch stubs from being emitted.)
typedef __attribute__((address_space(3))) void lds_void;
__device__ __forceinline__ void buf_to_lds16(rsrc_t r, uint8_t *lds, uint32_t voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void buf_to_lds4(rsrc_t r, uint8_t *lds, uint32_t voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 4, voff, soff, 0, 0);
}

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0], expcnt[6:4],
// lgkmcnt[11:8], vmcnt[5:4] at [15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier without the memory fence __syncthreads() adds (that
// fence would wait for every outstanding load, including the ones issued
// ahead for later stages).  The "memory" clobber keeps the compiler from
// moving loads and stores across it; completion of the copies a stage needs
// is waited for explicitly with wait_vmcnt before it.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Barrier after LDS writes only: waits for this wavefront's LDS accesses
// (lgkmcnt 0), not for its outstanding global loads.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
    asm volatile("s_barrier" ::: "memory");
}

// DPP lane permutations within a row of 16 lanes.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int DPP_QUAD_XOR1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;  // quad_perm [2,3,0,1]

// Sum over aligned groups of 4 lanes; every lane of the group gets the sum.
// All lanes of each group must be active.
__device__ __forceinline__ int quad_sum_i(int v) {
    v += dpp_i<DPP_QUAD_XOR1>(v);
    v += dpp_i<DPP_QUAD_XOR2>(v);
    return v;
}

// f16 -> f32 (exact; v_cvt_f32_f16 with f16 denormals preserved, the HIP
// default mode -- tests cover subnormal d values).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xffffu));
}

// IEEE binary32 -> binary16, round to nearest even (the `half` crate's
// from_f32), done on integers so it does not depend on the f16 denormal mode.
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
    uint32_t x = __float_as_uint(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u) | (man >> 13));
    int e = (int)exp - 112;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        int shift = 14 - e;
        if (shift > 24) return (uint16_t)sign;
        uint32_t m24 = man | 0x800000u;
        uint32_t r = m24 >> shift;
        uint32_t rem = m24 & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

// Rust `v as i8` for an integral-valued float: saturating, NaN -> 0.
__device__ __forceinline__ int sat_i8(float v) {
    if (v != v) return 0;
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    return (int)v;
}

__device__ __forceinline__ uint32_t pack4_i8(const int q[4]) {
    return (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) | ((uint32_t)(q[2] & 0xff) << 16) |
           ((uint32_t)(q[3] & 0xff) << 24);
}

constexpr int DPP_HALF_MIRROR = 0x141;  // lane i <-> 7-i within each 8 lanes
constexpr int DPP_ROW_MIRROR = 0x140;   // lane i <-> 15-i within each 16 lanes

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Wave-uniform max / min over all 64 lanes (all lanes active): max within
// each row of 16 lanes by DPP, then across the four rows by readlane.
__device__ __forceinline__ float wave_max_f(float v) {
    v = fmaxf(v, dpp_f<DPP_QUAD_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_QUAD_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_MIRROR>(v));
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}
__device__ __forceinline__ int wave_min_i(int v) {
    v = min(v, dpp_i<DPP_QUAD_XOR1>(v));
    v = min(v, dpp_i<DPP_QUAD_XOR2>(v));
    v = min(v, dpp_i<DPP_HALF_MIRROR>(v));
    v = min(v, dpp_i<DPP_ROW_MIRROR>(v));
    return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// One Q8_K block (candle-core 0.8.4 BlockQ8K::from_float) quantised by one
// full wavefront: lane l holds elements 4l..4l+3 in v.  Returns the four
// quants packed in a dword; *bsum gets the sum of the 16 quants of lanes
// 4(l/4)..4(l/4)+3 (every lane of the quad), *d the block's d (uniform).
// candle scans the block in order with `if amax < x.abs() { amax = |x|; max = x }`,
// so max is the FIRST element of largest |x| (NaN never wins); then
// iscale = -128/max, q = min(round(iscale*x), 127) with ties away from zero,
// d = 1/iscale; an all-zero block gives d = 0, q = 0.  Here: amax = max |x|
// over the wave, then the smallest index attaining it, then that element.
// IEEE division (the library is built without fast-math) keeps it bit-exact.
__device__ __forceinline__ uint32_t q8k_block_wave(const float v[4], int lane, int *bsum, float *d) {
    float ax[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a = fabsf(v[i]);
        ax[i] = a == a ? a : 0.0f;  // NaN never becomes the max
    }
    const float am = wave_max_f(fmaxf(fmaxf(ax[0], ax[1]), fmaxf(ax[2], ax[3])));
    int q[4] = {0, 0, 0, 0};
    float dd = 0.0f;
    if (am != 0.0f) {  // uniform
        int li = 1 << 30;
#pragma unroll
        for (int i = 3; i >= 0; i--)
            if (ax[i] == am) li = 4 * lane + i;
        const int idx = wave_min_i(li);
        const int c = idx & 3;
        const float mine = c == 0 ? v[0] : c == 1 ? v[1] : c == 2 ? v[2] : v[3];
        const float mx = readlane_f(mine, idx >> 2);
        const float iscale = -128.0f / mx;
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = sat_i8(fminf(roundf(iscale * v[i]), 127.0f));
        dd = 1.0f / iscale;
    }
    *bsum = quad_sum_i(q[0] + q[1] + q[2] + q[3]);
    *d = dd;
    return pack4_i8(q);
}

// One Q8_K block (candle-core 0.8.4 BlockQ8K::from_float) by the 16 lanes of a
// DPP row: lane s holds elements 16s..16s+15 in v.  Same arithmetic as
// q8k_block_wave: max = the first element of largest |x| (NaN
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
    m = fmaxf(m, dpp_f<DPP_QUAD_XOR1>(m));
    m = fmaxf(m, dpp_f<DPP_QUAD_XOR2>(m));
    m = fmaxf(m, dpp_f<DPP_HALF_MIRROR>(m));
    m = fmaxf(m, dpp_f<DPP_ROW_MIRROR>(m));
    int q[16];
    float dd = 0.0f;
    if (m != 0.0f) {  // uniform over the row
        int key = 1 << 30;
#pragma unroll
        for (int i = 15; i >= 0; i--)
            if (ax[i] == m) key = ((16 * s + i) << 1) | (v[i] < 0.0f ? 1 : 0);
        key = min(key, dpp_i<DPP_QUAD_XOR1>(key));
        key = min(key, dpp_i<DPP_QUAD_XOR2>(key));
        key = min(key, dpp_i<DPP_HALF_MIRROR>(key));
        key = min(key, dpp_i<DPP_ROW_MIRROR>(key));
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

// The stores of one Q8_K block by a wavefront (q8k_block_wave's layout):
// lane l writes quants 4l..4l+3 (and their f16 copy when a.q16 is set), the
// first lane of each quad its bsum, lane 0 d.  Block sb of row `row`, rows of
// k elements.
__device__ __forceinline__ void store_q8k_block64(const ActPlanes &a, int64_t row, int64_t k, int64_t sb, int lane,
                                                  uint32_t packed, int bsum, float d) {
    const int64_t e0 = row * k + sb * QK_K + 4 * lane;
    *(uint32_t *)(a.qs + e0) = packed;
    if (a.q16) {
        uint32_t o[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)(int)(int8_t)((packed >> (16 * j)) & 0xffu));
            const uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)(int)(int8_t)((packed >> (16 * j + 8)) & 0xffu));
            o[j] = lo | (hi << 16);
        }
        *(uint2 *)(a.q16 + e0) = make_uint2(o[0], o[1]);
    }
    if ((lane & 3) == 0) {
        a.bsums[row * (k / 16) + sb * 16 + (lane >> 2)] = (int16_t)bsum;
        a.bsum16[row * (k / 16) + sb * 16 + (lane >> 2)] = __builtin_bit_cast(uint16_t, (_Float16)(float)bsum);
    }
    if (lane == 0) a.d[row * (k / QK_K) + sb] = d;
}

// One Q8_0 block (BlockQ8_0::from_float) quantised by eight consecutive
// lanes (lane sub = l%8 holds elements 4sub..4sub+3): d = amax/127, id = 1/d
// (0 if d == 0), q = round(x*id) as i8, stored d = f16(d) (RNE).  Returns the
// packed quants; *d16 gets the f16 bits (uniform over the 8 lanes).  All 64
// lanes of the wave must be active.
__device__ __forceinline__ uint32_t q8_0_block_8lanes(const float v[4], uint16_t *d16) {
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) am = fmaxf(am, fabsf(v[i]));
    am = fmaxf(am, dpp_f<DPP_QUAD_XOR1>(am));
    am = fmaxf(am, dpp_f<DPP_QUAD_XOR2>(am));
    am = fmaxf(am, dpp_f<DPP_HALF_MIRROR>(am));
    const float d = am / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    int q[4];
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = sat_i8(roundf(v[i] * id));
    *d16 = f32_to_f16_rne(d);
    return pack4_i8(q);
}

// The same block quantised by two adjacent lanes (2j, 2j + 1 of a 16-lane
// set, 16 consecutive elements each; the row-per-lane matvec's prologue).
// Returns the 16 packed quants; *d16 gets the f16 bits (the same on both
// lanes).  All 64 lanes of the wave must be active.
__device__ __forceinline__ uint4 q8_0_block_2lanes(const float v[16], uint16_t *d16) {
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) am = fmaxf(am, fabsf(v[i]));
    am = fmaxf(am, dpp_f<DPP_QUAD_XOR1>(am));
    const float d = am / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    int q[16];
#pragma unroll
    for (int i = 0; i < 16; i++) q[i] = sat_i8(roundf(v[i] * id));
    *d16 = f32_to_f16_rne(d);
    return make_uint4(pack4_i8(q), pack4_i8(q + 4), pack4_i8(q + 8), pack4_i8(q + 12));
}

}  // namespace aq
#endif
