// decode_kernels.hip -- gfx950 device code for one BitNet-b1.58 decode step.
//
// One token at one position, the whole model device-resident: the order of
// src/forward.c:589-835 (n = 1), every float operation in the reference's
// order so that each intermediate carries the reference's bits, and therefore
// every int8 activation and every int32 dot of every layer does too. Built
// into its own code object (decode_gfx950.hsaco) and launched by decode.c.
//
// Launches per token (decode.c lays them out once per context):
//   per layer  sllm_k_dec_gemv   Q, K, V   (prologue: residual, attn_norm, quantise)
//              sllm_k_dec_scores           (RoPE, KV store, q . k)
//              sllm_k_dec_pv               (softmax, p . V)
//              sllm_k_dec_gemv   O         (prologue: attn_sub_norm, quantise)
//              sllm_k_dec_gemv   gate, up  (prologue: residual, ffn_norm, quantise;
//                                           epilogue: silu(gate) * up)
//              sllm_k_dec_gemv   down      (prologue: ffn_sub_norm, quantise)
//   then       sllm_k_dec_lm_head          (residual, output_norm, F16 rows)
//              sllm_k_dec_argmax           (argmax, next token)
//
// Floating-point contract: IEEE single and double, correctly rounded division
// and square root, no contraction (explicit fmaf where the reference calls an
// FMA), denormals kept -- the flags in the Makefile.

#include "i2s_device.h"
#include "libm_expf.h"

namespace {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x8 __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------------------
// device-resident state of a decode context (mirrored in decode.c)
// ---------------------------------------------------------------------------

struct dec_step {
    int32_t        token;       // the token the next step consumes
    int32_t        pos;         // its position
    int32_t        next;        // argmax of the last logits
    int32_t        advance;     // nonzero: the step moves on by itself (greedy loop)
    uint64_t       reserved0;
    uint32_t       reserved1;
    uint32_t       err;
    const int32_t *feed;        // prompt tokens still to consume: feed[i_feed .. n_feed)
    int32_t       *gen;         // generated tokens
    int32_t        n_feed, i_feed, n_gen, cap_gen;
};
static_assert(sizeof(dec_step) == 64, "dec_step must match decode.c");

// ---------------------------------------------------------------------------
// the reference's scalar operations
// ---------------------------------------------------------------------------

// binary16 -> binary32 as the token-embedding lookup converts
// (src/forward.c:239-262): exact except that a subnormal comes out at half
// its value (the lookup builds its exponent one too low).
__device__ __forceinline__ float embd_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16, ex = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    if (ex == 0) return __uint_as_float(__float_as_uint((float) man * 0x1p-25f) | sign);
    if (ex == 0x1fu) return __uint_as_float(sign | 0x7f800000u | (man << 13));
    return __uint_as_float(sign | ((ex + 112u) << 23) | (man << 13));
}

__constant__ uint64_t c_expf_tab[32] = SLLM_EXPF_TAB_INIT;

// Sum over the wave in double, as wave_sum (every lane gets it). The order
// of the additions is not the reference's: the callers' checks allow any.
template <int CTRL>
__device__ __forceinline__ double dpp_mov_d(double v) {
    return __hiloint2double(dpp_mov<CTRL>(__double2hiint(v)), dpp_mov<CTRL>(__double2loint(v)));
}

__device__ __forceinline__ double read_lane_d(double v, int lane) {
    return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), lane),
                            __builtin_amdgcn_readlane(__double2loint(v), lane));
}

__device__ __forceinline__ double wave_sum_d(double v) {
    v += dpp_mov_d<DPP_XOR1>(v);
    v += dpp_mov_d<DPP_XOR2>(v);
    v += dpp_mov_d<DPP_HALF_MIRROR>(v);
    v += dpp_mov_d<DPP_MIRROR>(v);
    return (read_lane_d(v, 0) + read_lane_d(v, 16)) + (read_lane_d(v, 32) + read_lane_d(v, 48));
}

// ---------------------------------------------------------------------------
// RMSNorm mean (src/ops.c:254-322)
// ---------------------------------------------------------------------------
//
// The reference sums the f32 squares in double over four lanes (lane l takes
// x[8i+l], then x[8i+4+l]), folds the lanes 0..3 and narrows sum/n to f32.
// Here the workgroup sums its threads' partials in any order. Both orders
// are sums of the same k nonnegative doubles, so they differ by at most
// (k + 64) * 2^-52 of the total; when every value in that interval narrows
// to the same f32 mean -- the narrowing is monotone, so checking the two
// ends suffices -- that f32 is the reference's. Otherwise (rarely: a mean
// within about 1e-12 relative of a rounding boundary) four threads run the
// reference's own lanes, re-reading the vector through elem(j).
// part: this thread's sum of (double)(x*x) over its elements; every thread
// of the block calls this. k % 8 == 0.
template <typename Elem>
__device__ float rms_mean(double part, uint32_t k, double *red_d, double *lane_d, Elem elem) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = (int) (blockDim.x >> 6);
    part = wave_sum_d(part);
    if (lane == 0) red_d[wave] = part;
    __syncthreads();
    double s = 0.0;
    for (int w = 0; w < nw; ++w) s += red_d[w];
    const double kd = (double) k;
    const double bound = s * ((double) (k + 64u) * 0x1p-52);
    const float lo = (float) ((s - bound) / kd), hi = (float) ((s + bound) / kd);
    float mean = lo;
    if (lo != hi) {                                  // uniform over the block
        if (tid < 4) {
            double acc = 0.0;
            for (uint32_t i = 0; i + 8 <= k; i += 8) {
                const float a = elem(i + (uint32_t) tid), b = elem(i + 4u + (uint32_t) tid);
                acc += (double) (a * a);
                acc += (double) (b * b);
            }
            lane_d[tid] = acc;
        }
        __syncthreads();
        double ss = 0.0;
        for (int l = 0; l < 4; ++l) ss += lane_d[l];
        mean = (float) (ss / kd);
    }
    __syncthreads();                                 // red_d / lane_d free again
    return mean;
}

// ---------------------------------------------------------------------------
// decode GEMV stage: a slab GEMV (the kernel of i2s_kernels.hip) whose
// workgroups first build the activation themselves -- residual add or
// embedding lookup, RMSNorm, quantisation -- so that no separate launch
// produces it. Every workgroup computes the same bits; workgroup 0 (flag
// WG_PUBLISH) writes what later launches need: the residual and, for
// tracing, the quantised row.
// ---------------------------------------------------------------------------

enum : uint32_t { IN_PLAIN = 0, IN_RESID = 1, IN_EMBED = 2 };

struct dec_stage {
    const void     *a;         // IN_PLAIN / IN_RESID: f32[k]; IN_EMBED: f16 rows [n_vocab][k]
    const float    *b;         // IN_RESID: added to a
    float          *v_out;     // the vector as built (before the norm), or null
    const float    *norm_w;    // RMSNorm weight, k floats
    const dec_step *step;      // IN_EMBED: the token
    int8_t         *q_out;     // the quantised row, or null
    act_t          *act_out;   // its scale / sum, or null
    float           eps;
    uint32_t        k;
    uint32_t        mode;
    uint32_t        pad;
};
static_assert(sizeof(dec_stage) == 72, "dec_stage must match decode.c");

struct dec_shared {
    int8_t  q[SLAB_MAX_K];
    int32_t dots[SLAB_MAX_ROWS];
    double  red_d[SLAB_WAVES];
    double  lane_d[4];
    float   red_f[SLAB_WAVES];
    int     red_i[SLAB_WAVES];
    int     red_a[SLAB_WAVES];
};

template <int MODE>
__device__ __forceinline__ float stage_elem(const dec_stage &st, int32_t token, uint32_t j) {
    if (MODE == IN_EMBED) return embd_f32(((const uint16_t *) st.a)[(size_t) token * st.k + j]);
    float v = ((const float *) st.a)[j];
    if (MODE == IN_RESID) v = v + st.b[j];
    return v;
}

template <int LPR, int CPL, int XV, int QV, int MODE, bool PAIR>
__device__ __forceinline__ void dec_block(const dec_stage &st, const gemv_job &job0, const gemv_job &job1,
                                          uint32_t slab, uint32_t n_slabs, uint32_t flags, dec_shared &S) {
    constexpr uint32_t RPW = 64 / LPR;
    constexpr uint32_t G = SLAB_WAVES * RPW;
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane((uint32_t) tid >> 6);
    const uint32_t k = job0.k, row_bytes = k >> 2;
    const uint32_t n_rows = job0.n_rows, last_row = n_rows - 1;
    const __amdgpu_buffer_rsrc_t rs0 = tensor_rsrc(job0), rs1 = tensor_rsrc(job1);
    const uint32_t n_groups = (n_rows + G - 1) / G;
    const uint32_t per = (n_groups + n_slabs - 1) / n_slabs;
    const uint32_t first = slab * per;
    const uint32_t T = first < n_groups ? min(per, n_groups - first) : 0u;
    if (T == 0) return;                               // uniform
    const uint32_t TT = PAIR ? 2 * T : T;             // groups: job0's, then job1's
    const uint32_t wave_row = wave * RPW;
    auto group_row = [&](uint32_t t) {
        const uint32_t i = min(t, TT - 1);
        return (first + (PAIR && i >= T ? i - T : i)) * G + wave_row;
    };
    auto group_rsrc = [&](uint32_t t) { return (PAIR && min(t, TT - 1) >= T) ? rs1 : rs0; };

    // (1) the input vector and the norm weight
    const int32_t token = MODE == IN_EMBED ? st.step->token : 0;
    f32x4 v[XV], nw[XV];
#pragma unroll
    for (int u = 0; u < XV; ++u) {
        const uint32_t i = min(4u * (uint32_t) (tid + u * SLAB_THREADS), k - 4);
        if (MODE == IN_EMBED) {
            const u32x2 h = *G_CAST(const u32x2, (const uint16_t *) st.a + (size_t) token * k + i);
            v[u] = (f32x4) { embd_f32(h[0] & 0xffffu), embd_f32(h[0] >> 16),
                             embd_f32(h[1] & 0xffffu), embd_f32(h[1] >> 16) };
        } else {
            f32x4 a = *G_CAST(const f32x4, (const float *) st.a + i);
            if (MODE == IN_RESID) a = a + *G_CAST(const f32x4, st.b + i);
            v[u] = a;
        }
        nw[u] = *G_CAST(const f32x4, st.norm_w + i);
    }
    const float ws0 = tensor_scale(job0);
    const float ws1 = PAIR ? tensor_scale(job1) : 0.0f;
    __builtin_amdgcn_sched_barrier(0);

    // (2) the first weight group streams while the activation is built
    u32x4 bufa[CPL], bufb[CPL];
    slab_load<LPR, CPL>(group_rsrc(0), row_bytes, group_row(0), last_row, bufa);

    // (3) RMSNorm: mean of squares, scale = 1/sqrtf(mean + eps), (scale*x)*w
    double part = 0.0;
#pragma unroll
    for (int u = 0; u < XV; ++u) {
        if (4u * (uint32_t) (tid + u * SLAB_THREADS) < k) {
#pragma unroll
            for (int c = 0; c < 4; ++c) part += (double) (v[u][c] * v[u][c]);
        }
    }
    const float mean = rms_mean(part, k, S.red_d, S.lane_d,
                                [&](uint32_t j) { return stage_elem<MODE>(st, token, j); });
    const float scale = 1.0f / sqrtf(mean + st.eps);
    f32x4 xn[XV];
#pragma unroll
    for (int u = 0; u < XV; ++u) {
#pragma unroll
        for (int c = 0; c < 4; ++c) xn[u][c] = (scale * v[u][c]) * nw[u][c];
    }

    // (4) quantise (src/i2s_gemm.c:45-83) into LDS
    float m = 0.0f;
#pragma unroll
    for (int u = 0; u < XV; ++u) {
        const uint32_t i = 4u * (uint32_t) (tid + u * SLAB_THREADS);
        const float a = fmaxf(fmaxf(fabsf(xn[u][0]), fabsf(xn[u][1])), fmaxf(fabsf(xn[u][2]), fabsf(xn[u][3])));
        m = fmaxf(m, i < k ? a : 0.0f);
    }
    m = wave_max(m);
    if (lane == 0) S.red_f[wave] = m;
    __syncthreads();
    m = S.red_f[0];
#pragma unroll
    for (int w = 1; w < SLAB_WAVES; ++w) m = fmaxf(m, S.red_f[w]);
    const float qs = m > 0.0f ? 127.0f / m : 0.0f;
    int ls = 0, la = 0;
#pragma unroll
    for (int u = 0; u < XV; ++u) {
        const uint32_t i = 4u * (uint32_t) (tid + u * SLAB_THREADS);
        if (i < k) {
            const int a = quant_one(xn[u][0] * qs), b = quant_one(xn[u][1] * qs);
            const int c = quant_one(xn[u][2] * qs), e = quant_one(xn[u][3] * qs);
            ls += a + b + c + e;
            la += ((i >> 5) & 3u) == 0 ? a + b + c + e : 0;     // field 0 of its block
            *reinterpret_cast<uint32_t *>(S.q + i) =
                (uint32_t) (a & 0xff) | ((uint32_t) (b & 0xff) << 8) |
                ((uint32_t) (c & 0xff) << 16) | ((uint32_t) (e & 0xff) << 24);
        } else {
            *reinterpret_cast<uint32_t *>(S.q + i) = 0u;       // the dots' slots past the row
        }
    }
    ls = wave_sum(ls);
    la = wave_sum(la);
    if (lane == 0) {
        S.red_i[wave] = ls;
        S.red_a[wave] = la;
    }
    __syncthreads();
    int32_t asum = 0, a2 = 0;       // a2: twice the sum of the row's field-0 elements (slab_dot_x)
#pragma unroll
    for (int w = 0; w < SLAB_WAVES; ++w) {
        asum += S.red_i[w];
        a2 += 2 * S.red_a[w];
    }

    // (5) the row groups, double-buffered (as the slab kernel; the load past
    // the last group goes to the dead offset)
    int32_t *dots = S.dots + wave_row;
    uint32_t t = 0;
    for (uint32_t pair = 0; pair < TT / 2; ++pair) {
        slab_load<LPR, CPL>(group_rsrc(t + 1), row_bytes, group_row(t + 1), last_row, bufb, t + 1 < TT);
        slab_dot_x<LPR, CPL>(group_row(t), n_rows, bufa, S.q, a2, dots + t * G);
        ++t;
        slab_load<LPR, CPL>(group_rsrc(t + 1), row_bytes, group_row(t + 1), last_row, bufa, t + 1 < TT);
        slab_dot_x<LPR, CPL>(group_row(t), n_rows, bufb, S.q, a2, dots + t * G);
        ++t;
    }
    if (TT & 1u) slab_dot_x<LPR, CPL>(group_row(t), n_rows, bufa, S.q, a2, dots + t * G);
    __syncthreads();

    // (6) epilogue (src/forward.c:653-792): (float)(dot - sum) * (w_scale / act_scale);
    // gate / up: silu(gate) * up (src/forward.c:776-778)
    const float post0 = ws0 / qs;
    const float post1 = PAIR ? ws1 / qs : 0.0f;
    for (uint32_t i = (uint32_t) tid; i < T * G; i += SLAB_THREADS) {
        const uint32_t row = first * G + i;
        if (row < n_rows) {
            const int32_t d0 = S.dots[i];
            if (job0.out_i != nullptr) G_CAST(int32_t, job0.out_i)[row] = d0;
            float y = (float) (d0 - asum) * post0;
            if (PAIR) {
                const int32_t d1 = S.dots[T * G + i];
                if (job1.out_i != nullptr) G_CAST(int32_t, job1.out_i)[row] = d1;
                const float up = (float) (d1 - asum) * post1;
                y = silu(y) * up;
            }
            if (job0.out_f != nullptr) G_CAST(float, job0.out_f)[row] = y;
        }
    }

    // (7) workgroup 0 publishes the residual and the quantised row
    if (flags & WG_PUBLISH) {
#pragma unroll
        for (int u = 0; u < XV; ++u) {
            const uint32_t i = 4u * (uint32_t) (tid + u * SLAB_THREADS);
            if (i < k && st.v_out != nullptr) *G_CAST(f32x4, st.v_out + i) = v[u];
            if (i < k && st.q_out != nullptr) *G_CAST(uint32_t, st.q_out + i) = *reinterpret_cast<const uint32_t *>(S.q + i);
        }
        if (tid == 0 && st.act_out != nullptr) {
            G_CAST(float, st.act_out)[0] = qs;
            G_CAST(int32_t, st.act_out)[1] = asum;
        }
    }
}

// A decode GEMV stage as kernel arguments: the activation's recipe and up
// to three jobs sharing it (Q, K, V), or gate and up as one pair. Workgroup
// b (after the XCD remap) takes slab b of job 0, then job 1's, then job 2's;
// with a pair, job 1 has no slabs of its own.
struct dec_gemv_args {
    dec_stage st;
    gemv_job  job[3];
    uint32_t  n_slabs[3];
    uint32_t  n_wg;            // the grid, a multiple of 8
    uint32_t  pair;            // jobs 0 and 1 are gate and up
    uint32_t  pad[3];
};
static_assert(sizeof(dec_gemv_args) == 296, "dec_gemv_args must match decode.c");

template <int LPR, int CPL, int XV, int QV>
__device__ __forceinline__ void dec_variant(const dec_stage &st, const gemv_job &job0, const gemv_job &job1,
                                            bool pair, uint32_t slab, uint32_t n_slabs, uint32_t flags,
                                            dec_shared &S) {
    switch (st.mode) {
    case IN_EMBED:
        if (pair) dec_block<LPR, CPL, XV, QV, IN_EMBED, true>(st, job0, job1, slab, n_slabs, flags, S);
        else dec_block<LPR, CPL, XV, QV, IN_EMBED, false>(st, job0, job0, slab, n_slabs, flags, S);
        break;
    case IN_RESID:
        if (pair) dec_block<LPR, CPL, XV, QV, IN_RESID, true>(st, job0, job1, slab, n_slabs, flags, S);
        else dec_block<LPR, CPL, XV, QV, IN_RESID, false>(st, job0, job0, slab, n_slabs, flags, S);
        break;
    default:
        if (pair) dec_block<LPR, CPL, XV, QV, IN_PLAIN, true>(st, job0, job1, slab, n_slabs, flags, S);
        else dec_block<LPR, CPL, XV, QV, IN_PLAIN, false>(st, job0, job0, slab, n_slabs, flags, S);
        break;
    }
}

// ---------------------------------------------------------------------------
// attention (src/forward.c:668-726): RoPE (NeoX pairs, cos/sin from a table
// the host builds with the reference's libm calls), KV store, scores.
// ---------------------------------------------------------------------------

struct dec_attn {
    const float    *q, *k, *v;          // projections: q [n_head*hd], k / v [n_kv*hd]
    float          *k_cache;            // this layer's keys [n_kv][hd / 8][n_ctx][8]
    float          *v_cache;            // this layer's values [n_kv][hd / 8][n_ctx][8]: a slice of
                                        // eight dimensions of every position is contiguous
    const float    *rope;               // [n_ctx][half] (cos, sin)
    float          *scores;             // [n_head][sc_stride]
    float          *out;                // [n_head*hd]
    const dec_step *step;
    float           attn_scale;
    uint32_t        n_head, n_kv, hd, half, n_ctx;
    uint32_t        sc_stride;          // scores row stride: n_ctx rounded up to 8
    uint32_t        chunk_base;         // chunk kernels: the position of the chunk's first token
    const uint8_t  *ahead;              // chunk scores: bytes read ahead (this layer's O weights ..
    uint64_t        ahead_bytes;        // the next layer's V weights), a multiple of 16
};
static_assert(sizeof(dec_attn) == 120, "dec_attn must match decode.c");

constexpr int ATT_THREADS = 256;
constexpr uint32_t ATT_POS = 64;        // positions per scores workgroup
constexpr uint32_t ATT_MAX_HD = 128;
constexpr uint32_t ATT_MAX_GRP = 4;     // query heads per KV head
constexpr uint32_t KT_STRIDE = ATT_MAX_HD + 4;     // LDS key row: 16-byte aligned, rows 4 banks apart
constexpr int KT_LOADS = ATT_POS * ATT_MAX_HD / 4 / ATT_THREADS;   // float4 per thread
constexpr uint32_t PV_SLICE = 8;       // head dimensions per p.V workgroup
constexpr uint32_t PV_RPOS = 1536;      // positions of p (LDS) and V (registers) per round
constexpr uint32_t PV_SUB = 192;        // positions per product sub-round
constexpr uint32_t PV_XSTRIDE = PV_SUB + 4;                // LDS product row: rows 4 banks apart
constexpr int PV_THREADS = 512;                            // p.V workgroup: eight waves
constexpr int PV_WAVES = PV_THREADS / 64;
constexpr uint32_t PV_HPW = 2;                             // query heads per p.V workgroup
constexpr int PV_WPH = PV_WAVES / (int) PV_HPW;            // waves per head
constexpr uint32_t PV_SPAN = 512u * PV_WPH;                // positions of one pass: a group per lane
constexpr int PV_PTHREADS = 128;                           // producer threads: waves 3 and 7
constexpr int PV_VLOADS = (int) (PV_RPOS * PV_SLICE / 4 / PV_PTHREADS);   // float4 of V per producer
constexpr int PV_VSUB = (int) (PV_SUB * PV_SLICE / 4 / PV_PTHREADS);      // of them per sub-round
constexpr uint32_t PV_G4 = PV_SLICE / 4;                   // float4 per position of a slice
static_assert(ATT_MAX_GRP * PV_SLICE <= 64, "one chain wave");
static_assert(PV_VLOADS * PV_PTHREADS * 4 == (int) (PV_RPOS * PV_SLICE), "whole float4 per producer");
static_assert(PV_VSUB * PV_PTHREADS * 4 == (int) (PV_SUB * PV_SLICE) && PV_RPOS % PV_SUB == 0, "sub-rounds");
static_assert(PV_PTHREADS % PV_G4 == 0, "a producer keeps its dimensions");
static_assert(PV_SPAN >= PV_RPOS && PV_HPW * PV_SLICE <= 64, "one group per lane; one chain wave");

// NeoX RoPE (src/ops.c:467-549) of element d of a head vector: pairs
// (e, e + half) rotate by angle e, x[e] -> x[e] c - x[e+half] s and
// x[e+half] -> x[e] s + x[e+half] c; dimensions from 2*half on pass through.
// The operands are loaded first (rope_load, no branches around the loads),
// the arithmetic applied afterwards (rope_apply).
struct rope_in {
    float x, partner, c, s;
};

__device__ __forceinline__ rope_in rope_load(const float *x, uint32_t d, uint32_t half, const float *cs) {
    const uint32_t e = d < half ? d : (d < 2 * half ? d - half : 0);
    const uint32_t partner = d < half ? d + half : (d < 2 * half ? d - half : d);
    return { x[d], x[partner], cs[2 * e], cs[2 * e + 1] };
}

__device__ __forceinline__ float rope_apply(const rope_in &r, uint32_t d, uint32_t half) {
    if (d < half) return r.x * r.c - r.partner * r.s;
    if (d < 2 * half) return r.partner * r.s + r.x * r.c;
    return r.x;
}

constexpr int QR_PER_THREAD = (int) (ATT_MAX_GRP * ATT_MAX_HD / ATT_THREADS);

} // namespace

// ---------------------------------------------------------------------------
// entry points (argument lists mirrored in decode.c)
// ---------------------------------------------------------------------------

// One decode GEMV stage. Variant 0 (K <= 2560): 8 lanes per row; variant 1
// (K <= 7168): 16 lanes per row. Everything a workgroup needs arrives in the
// kernel arguments, so its first loads are the activation and the weights.
extern "C" __global__ void __launch_bounds__(SLAB_THREADS)
sllm_k_dec_gemv(dec_gemv_args A) {
    __shared__ dec_shared S;
    const uint32_t b = xcd_slot(A.n_wg);
    const uint32_t n0 = A.n_slabs[0], n01 = n0 + A.n_slabs[1], n012 = n01 + A.n_slabs[2];
    if (b >= n012) return;
    const uint32_t ji = b < n0 ? 0u : (b < n01 ? 1u : 2u);
    const uint32_t slab = b - (ji == 0 ? 0u : (ji == 1 ? n0 : n01));
    const gemv_job job0 = ji == 0 ? A.job[0] : (ji == 1 ? A.job[1] : A.job[2]);
    const gemv_job job1 = A.job[1];
    const uint32_t n_slabs = A.n_slabs[ji];
    const uint32_t flags = b == 0 ? WG_PUBLISH : 0u;
    const bool pair = A.pair != 0;
    if (job0.variant == 0) dec_variant<8, 5, 3, 1>(A.st, job0, job1, pair, slab, n_slabs, flags, S);
    else dec_variant<16, 7, 7, 2>(A.st, job0, job1, pair, slab, n_slabs, flags, S);
}

// Scores: workgroup (KV head, 64 positions). Every workgroup ropes the query
// heads of its KV head; in a decode step the one holding position pos ropes
// the new key and stores it, with the new value, into the caches
// (src/forward.c:668-690). Thread (h, r) then takes q_h . k_r over d in
// order, times 1/sqrt(hd) (src/forward.c:698-705). The cached keys are
// loaded first, all at once, and wait in registers while the queries are
// roped. CHUNK: grid z is the chunk's token t at position chunk_base + t,
// whose keys (its own included) are already in the cache; q, scores and out
// advance by one token's worth per t.
// The block of ATT_POS key rows from s0 as float4 f = 0 .. ATT_POS hd / 4 - 1
// of a workgroup's loads: f / 2 walks the rows of one eight-dimension slice
// of the cache, then the next slice, so that consecutive threads read
// consecutive 16 bytes; rows past `last` re-read row `last`. kt_src: the
// float offset in the KV head's cache; kt_col: the column in an LDS row.
__device__ __forceinline__ size_t kt_src(uint32_t f, uint32_t s0, uint32_t last, uint32_t n_ctx) {
    const uint32_t h2 = f & 1u, r = (f >> 1) % ATT_POS, sl = (f >> 1) / ATT_POS;
    return ((size_t) sl * n_ctx + min(s0 + r, last)) * PV_SLICE + 4u * h2;
}
__device__ __forceinline__ uint32_t kt_col(uint32_t f) { return ((f >> 1) / ATT_POS) * PV_SLICE + 4u * (f & 1u); }

template <bool CHUNK>
__device__ __forceinline__ void scores_body(const dec_attn &A) {
    __shared__ __attribute__((aligned(16))) float qr[ATT_MAX_GRP][ATT_MAX_HD];
    __shared__ __attribute__((aligned(16))) float kt[ATT_POS][KT_STRIDE];
    // decode step, at most eight KV heads: a one-dimensional grid of eight
    // columns, KV head h in column h (workgroups go to the eight XCDs in
    // turn), so that the scores land in the L2 of the XCD whose p.V
    // workgroups read them; the other columns return at once
    const bool xcd = !CHUNK && A.n_kv <= 8;
    const uint32_t kvh = xcd ? blockIdx.x % 8u : blockIdx.x;
    const uint32_t s0 = (xcd ? blockIdx.x / 8u : blockIdx.y) * ATT_POS, tid = threadIdx.x;
    if (kvh >= A.n_kv) return;
    const uint32_t t = CHUNK ? blockIdx.z : 0u;
    const uint32_t pos = CHUNK ? A.chunk_base + t : (uint32_t) A.step->pos, npast = pos + 1;
    if (s0 >= npast) return;
    const uint32_t grp = A.n_head / A.n_kv, hd = A.hd, half = A.half, hd4 = hd / 4;
    float *kc = A.k_cache + (size_t) kvh * A.n_ctx * hd;
    float *vc = A.v_cache + (size_t) kvh * A.n_ctx * hd;               // this KV head's value slices
    const float *cs = A.rope + (size_t) pos * (half > 0 ? half : 1) * 2;
    const float *q = A.q + (size_t) t * A.n_head * hd;
    float *scores = A.scores + (size_t) t * A.n_head * A.sc_stride;

    // (1) every global load first: the cached keys (rows past the last
    // cached one re-read a valid row), this thread's query elements and, in
    // a decode step, the new key's
    const uint32_t n_cached = CHUNK ? npast : pos;
    const uint32_t n_f4 = ATT_POS * hd4, last_cached = n_cached > 0 ? n_cached - 1 : 0;
    f32x4 kv[KT_LOADS];
#pragma unroll
    for (int u = 0; u < KT_LOADS; ++u) {
        const uint32_t f = min(tid + (uint32_t) u * ATT_THREADS, n_f4 - 1);
        kv[u] = *G_CAST(const f32x4, kc + kt_src(f, s0, last_cached, A.n_ctx));
    }
    rope_in qi[QR_PER_THREAD];
#pragma unroll
    for (int u = 0; u < QR_PER_THREAD; ++u) {
        const uint32_t idx = min(tid + (uint32_t) u * ATT_THREADS, grp * hd - 1);
        qi[u] = rope_load(q + (size_t) (kvh * grp + idx / hd) * hd, idx % hd, half, cs);
    }
    rope_in ki = {};
    float vnew = 0.0f;
    if (!CHUNK) {
        ki = rope_load(A.k + (size_t) kvh * hd, min(tid, hd - 1), half, cs);
        vnew = A.v[(size_t) kvh * hd + min(tid, hd - 1)];
    }

    // (2) roped queries, the new key and value, the cached keys into LDS
#pragma unroll
    for (int u = 0; u < QR_PER_THREAD; ++u) {
        const uint32_t idx = tid + (uint32_t) u * ATT_THREADS;
        if (idx < grp * hd) qr[idx / hd][idx % hd] = rope_apply(qi[u], idx % hd, half);
    }
    if (!CHUNK && pos - s0 < ATT_POS && tid < hd) {
        const float val = rope_apply(ki, tid, half);
        const size_t at = ((size_t) (tid / PV_SLICE) * A.n_ctx + pos) * PV_SLICE + tid % PV_SLICE;
        kt[pos - s0][tid] = val;
        kc[at] = val;
        vc[at] = vnew;
    }
#pragma unroll
    for (int u = 0; u < KT_LOADS; ++u) {
        const uint32_t f = tid + (uint32_t) u * ATT_THREADS, r = (f >> 1) % ATT_POS;
        if (f < n_f4 && s0 + r < n_cached) *reinterpret_cast<f32x4 *>(&kt[r][kt_col(f)]) = kv[u];
    }
    __syncthreads();
    // (3) thread (h, r): the dot in order of d
    const uint32_t r = tid % ATT_POS, hh = tid / ATT_POS;
    if (r < min(ATT_POS, npast - s0) && hh < grp) {
        float acc = 0.0f;
        for (uint32_t d4 = 0; d4 < hd4; ++d4) {
            const f32x4 k4 = *reinterpret_cast<const f32x4 *>(&kt[r][4 * d4]);
            const f32x4 q4 = *reinterpret_cast<const f32x4 *>(&qr[hh][4 * d4]);
            acc = acc + q4[0] * k4[0];
            acc = acc + q4[1] * k4[1];
            acc = acc + q4[2] * k4[2];
            acc = acc + q4[3] * k4[3];
        }
        scores[(size_t) (kvh * grp + hh) * A.sc_stride + s0 + r] = acc * A.attn_scale;
    }
}

extern "C" __global__ void __launch_bounds__(ATT_THREADS)
sllm_k_dec_scores(dec_attn A) { scores_body<false>(A); }

// The chunk's scores: workgroup (KV head, 64 positions, TOK tokens), so
// that a block of cached keys, loaded once into LDS, serves TOK tokens (8;
// 4 for small chunks, whose grid would otherwise be a few dozen). Thread
// (h, r) -- wave h is query head h of the KV head, lane r a position --
// holds TOK dot chains: token by token the q . k of the decode kernel, in
// order of d, times 1/sqrt(hd), written for the positions at or before each
// token's own. The queries were roped at their positions by
// sllm_k_chk_kv_store; they are the same for every lane of a wave and come
// through the scalar unit (8 dimensions of a token per load), so the LDS
// serves only the keys.
typedef float f32x8 __attribute__((ext_vector_type(8)));

template <uint32_t CS_TOK, uint32_t NB = 1>
__device__ __forceinline__ void chk_scores_body(const dec_attn &A, uint32_t n_tok) {
    constexpr uint32_t THREADS = ATT_THREADS * NB, LOADS = KT_LOADS / NB;   // NB token blocks per workgroup
    __shared__ __attribute__((aligned(16))) float kt[ATT_POS][KT_STRIDE];
    const uint32_t kvh = blockIdx.x, s0 = blockIdx.y * ATT_POS, tb0 = blockIdx.z * CS_TOK * NB, tid = threadIdx.x;
    const uint32_t npast_wg = A.chunk_base + min(tb0 + CS_TOK * NB, n_tok);   // of the workgroup's last token
    if (s0 >= npast_wg) return;
    const uint32_t grp = A.n_head / A.n_kv, hd = A.hd, hd4 = hd / 4;
    const float *kc = A.k_cache + (size_t) kvh * A.n_ctx * hd;

    // the block's keys (rows past the last token's position re-read a valid row)
    const uint32_t n_f4 = ATT_POS * hd4, last_cached = npast_wg - 1;
    f32x4 kv[LOADS];
#pragma unroll
    for (int u = 0; u < (int) LOADS; ++u) {
        const uint32_t f = min(tid + (uint32_t) u * THREADS, n_f4 - 1);
        kv[u] = *G_CAST(const f32x4, kc + kt_src(f, s0, last_cached, A.n_ctx));
    }
#pragma unroll
    for (int u = 0; u < (int) LOADS; ++u) {
        const uint32_t f = tid + (uint32_t) u * THREADS, r = (f >> 1) % ATT_POS;
        if (f < n_f4 && s0 + r < npast_wg) *reinterpret_cast<f32x4 *>(&kt[r][kt_col(f)]) = kv[u];
    }
    __syncthreads();

    // wave w: query head w % 4 of the KV head, token block w / 4 of the workgroup's NB
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / ATT_POS), r = tid % ATT_POS, hh = wave % 4u;
    const uint32_t tb = tb0 + (wave / 4u) * CS_TOK;
    if (hh >= grp || tb >= n_tok) return;            // uniform; no barriers past this point
    const uint32_t last_tok = min(tb + CS_TOK, n_tok) - 1;
    const uint32_t npast_max = A.chunk_base + last_tok + 1;
    if (s0 >= npast_max) return;                     // no position of this block at or before its tokens
    // the queries are not written during the launch: constant address
    // space, so that their wave-uniform reads are scalar loads
    typedef __attribute__((address_space(4))) const float cfloat;
    typedef __attribute__((address_space(4))) const f32x4 cf32x4;
    cfloat *qrow[CS_TOK];
#pragma unroll
    for (int tk = 0; tk < (int) CS_TOK; ++tk)
        qrow[tk] = (cfloat *) (A.q + ((size_t) min(tb + (uint32_t) tk, last_tok) * A.n_head + kvh * grp + hh) * hd);
    float acc[CS_TOK];
#pragma unroll
    for (int tk = 0; tk < (int) CS_TOK; ++tk) acc[tk] = 0.0f;
    // four dimensions per step. The queries of the next step load while
    // this one computes: scalar loads return out of order, so a wait covers
    // all of them, and the next step's loads go out only after this step's
    // first product has waited for its own (two buffers of CS_TOK x 4 words)
    auto qload = [&](uint32_t d0, f32x4 (&q)[CS_TOK]) {
#pragma unroll
        for (int tk = 0; tk < (int) CS_TOK; ++tk) q[tk] = *(cf32x4 *) (qrow[tk] + min(d0, hd - 4));
    };
    auto step4 = [&](uint32_t d0, const f32x4 (&qc)[CS_TOK], f32x4 (&qn)[CS_TOK]) {
        const f32x4 k4 = *reinterpret_cast<const f32x4 *>(&kt[r][d0]);
        float a0 = acc[0] + qc[0][0] * k4[0];
        __builtin_amdgcn_sched_barrier(0);
        qload(d0 + 4, qn);
        __builtin_amdgcn_sched_barrier(0);
        a0 = a0 + qc[0][1] * k4[1];
        a0 = a0 + qc[0][2] * k4[2];
        acc[0] = a0 + qc[0][3] * k4[3];
#pragma unroll
        for (int tk = 1; tk < (int) CS_TOK; ++tk) {
            float a = acc[tk];
            a = a + qc[tk][0] * k4[0];
            a = a + qc[tk][1] * k4[1];
            a = a + qc[tk][2] * k4[2];
            acc[tk] = a + qc[tk][3] * k4[3];
        }
    };
    f32x4 qa[CS_TOK], qb[CS_TOK];
    qload(0, qa);
    for (uint32_t d0 = 0; d0 < hd; d0 += 8) {       // hd % 8 == 0
        step4(d0, qa, qb);
        step4(d0 + 4, qb, qa);
    }
    if (s0 + r < npast_max) {
#pragma unroll
        for (int tk = 0; tk < (int) CS_TOK; ++tk) {
            const uint32_t t = tb + (uint32_t) tk;
            if (t < n_tok && s0 + r <= A.chunk_base + t) {
                A.scores[(size_t) t * A.n_head * A.sc_stride + (size_t) (kvh * grp + hh) * A.sc_stride + s0 + r] =
                    acc[tk] * A.attn_scale;
            }
        }
    }
}

extern "C" __global__ void __launch_bounds__(ATT_THREADS)
sllm_k_chk_scores(dec_attn A, uint32_t n_tok) { chk_scores_body<8>(A, n_tok); }
extern "C" __global__ void __launch_bounds__(ATT_THREADS)
sllm_k_chk_scores4(dec_attn A, uint32_t n_tok) { chk_scores_body<4>(A, n_tok); }

// The chunk's scores as units of one wave: (KV head, query head, 8 tokens,
// 64 positions), lane r = position s0 + r, the same dot chains as above.
// The lane streams its key from the cache (L2) in chunks of 32 dimensions
// (four slices of eight: each load instruction reads 16 bytes of 64
// consecutive positions, 32 bytes apart, rather than 64 separate rows), the
// next chunk in flight while this one is used, so the wave needs no LDS and
// no barrier; the queries come
// through the scalar unit as above, the next step's in flight. A
// workgroup of sixteen waves runs on each CU (the host pads its LDS so that
// no second one fits) and takes units cu, cu + G, cu + 2G, ... of the
// launch's G workgroups, so that every CU has the same number of units to
// within one, at most one more than the others on each SIMD.
constexpr int CSW_THREADS = 1024;
constexpr uint32_t CSW_TOK = 8;

__device__ __forceinline__ void chk_scores_unit(const dec_attn &A, uint32_t n_tok, uint32_t kvh, uint32_t hh,
                                                uint32_t tb, uint32_t s0, uint32_t lane) {
    const uint32_t grp = A.n_head / A.n_kv, hd = A.hd;
    const uint32_t last_tok = min(tb + CSW_TOK, n_tok) - 1;
    const uint32_t npast_max = A.chunk_base + last_tok + 1;
    // the lane's key (rows past the last token's position re-read a valid
    // row): eight dimensions at krow, the next eight n_ctx * 8 floats on
    const GLOBAL float *krow = G_CAST(const float, A.k_cache + ((size_t) kvh * A.n_ctx * hd +
                                                                (size_t) min(s0 + lane, npast_max - 1) * PV_SLICE));
    const size_t kslice = (size_t) A.n_ctx * PV_SLICE;
    typedef __attribute__((address_space(4))) const float cfloat;
    typedef __attribute__((address_space(4))) const f32x4 cf32x4;
    cfloat *qrow[CSW_TOK];
#pragma unroll
    for (int tk = 0; tk < (int) CSW_TOK; ++tk)
        qrow[tk] = (cfloat *) (A.q + ((size_t) min(tb + (uint32_t) tk, last_tok) * A.n_head + kvh * grp + hh) * hd);
    float acc[CSW_TOK];
#pragma unroll
    for (int tk = 0; tk < (int) CSW_TOK; ++tk) acc[tk] = 0.0f;
    auto qload = [&](uint32_t d0, f32x4 (&q)[CSW_TOK]) {
#pragma unroll
        for (int tk = 0; tk < (int) CSW_TOK; ++tk) q[tk] = *(cf32x4 *) (qrow[tk] + min(d0, hd - 4));
    };
    // four dimensions: the first product waits for this step's queries, then
    // the next step's go out
    auto step4 = [&](uint32_t d0, const f32x4 &k4, const f32x4 (&qc)[CSW_TOK], f32x4 (&qn)[CSW_TOK]) {
        float a0 = acc[0] + qc[0][0] * k4[0];
        __builtin_amdgcn_sched_barrier(0);
        qload(d0 + 4, qn);
        __builtin_amdgcn_sched_barrier(0);
        a0 = a0 + qc[0][1] * k4[1];
        a0 = a0 + qc[0][2] * k4[2];
        acc[0] = a0 + qc[0][3] * k4[3];
#pragma unroll
        for (int tk = 1; tk < (int) CSW_TOK; ++tk) {
            float a = acc[tk];
            a = a + qc[tk][0] * k4[0];
            a = a + qc[tk][1] * k4[1];
            a = a + qc[tk][2] * k4[2];
            acc[tk] = a + qc[tk][3] * k4[3];
        }
    };
    const uint32_t n_ch = hd / 32u;                    // hd % 32 == 0
    auto kload = [&](uint32_t ch, f32x4 (&k)[8]) {
        const uint32_t sl = min(ch, n_ch - 1u) * 4u;     // four slices of eight dimensions
#pragma unroll
        for (int i = 0; i < 8; ++i)
            k[i] = *reinterpret_cast<const GLOBAL f32x4 *>(krow + (sl + (uint32_t) i / 2u) * kslice + 4u * ((uint32_t) i & 1u));
    };
    // 32 dimensions; queries of its first step in qa on entry, of the next chunk's first step on exit
    f32x4 qa[CSW_TOK], qb[CSW_TOK];
    auto chunk = [&](uint32_t ch, const f32x4 (&k)[8]) {
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            step4(32u * ch + 4u * (uint32_t) i, k[i], qa, qb);
            step4(32u * ch + 4u * (uint32_t) i + 4u, k[i + 1], qb, qa);
        }
    };
    f32x4 ka[8], kb[8];
    kload(0, ka);
    qload(0, qa);
    kload(1, kb);
    uint32_t ch = 0;
    for (; ch + 2 <= n_ch; ch += 2) {
        chunk(ch, ka);
        kload(ch + 2, ka);
        chunk(ch + 1, kb);
        kload(ch + 3, kb);
    }
    if (ch < n_ch) chunk(ch, ka);                      // an odd chunk count
    if (s0 + lane < npast_max) {
#pragma unroll
        for (int tk = 0; tk < (int) CSW_TOK; ++tk) {
            const uint32_t t = tb + (uint32_t) tk;
            if (t < n_tok && s0 + lane <= A.chunk_base + t) {
                A.scores[(size_t) t * A.n_head * A.sc_stride + (size_t) (kvh * grp + hh) * A.sc_stride + s0 + lane] =
                    acc[tk] * A.attn_scale;
            }
        }
    }
}

extern "C" __global__ void __launch_bounds__(CSW_THREADS)
sllm_k_chk_scores_w(dec_attn A, uint32_t n_tok) {
    // the GEMMs that follow read their weights from HBM with few loads in
    // flight; this VALU-bound kernel leaves the bandwidth idle, so it reads
    // them first (five 16-byte loads per thread over the whole grid, used
    // only at the end): they then come from the Infinity Cache
    constexpr int AHEAD = 5;
    u32x4 ahead[AHEAD];
    {
        const size_t n16 = A.ahead_bytes / 16, stride = (size_t) gridDim.x * CSW_THREADS;
        const GLOBAL u32x4 *src = G_CAST(const u32x4, A.ahead);
#pragma unroll
        for (int j = 0; j < AHEAD; ++j) {
            const size_t at = (size_t) blockIdx.x * CSW_THREADS + threadIdx.x + (size_t) j * stride;
            ahead[j] = at < n16 ? src[at] : (u32x4) { 0u, 0u, 0u, 0u };
        }
    }
    const uint32_t lane = threadIdx.x & 63u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t G = gridDim.x, cu = blockIdx.x, nkh = A.n_head;
    const uint32_t grp = A.n_head / A.n_kv;
    // lane j: token block j's position blocks (a chunk has at most 512
    // tokens: 64 blocks), then their inclusive prefix sum over the lanes
    const uint32_t n_tb = (n_tok + CSW_TOK - 1) / CSW_TOK;
    uint32_t inc = lane < n_tb ? (A.chunk_base + min(CSW_TOK * (lane + 1u), n_tok) + ATT_POS - 1) / ATT_POS : 0u;
#pragma unroll
    for (int o = 1; o < 64; o *= 2) {
        const uint32_t up = (uint32_t) __shfl_up((int) inc, (unsigned) o);
        inc += lane >= (uint32_t) o ? up : 0u;
    }
    const uint32_t n_pairs = __builtin_amdgcn_readlane(inc, 63);
    const uint32_t n_units = n_pairs * nkh;
    for (uint32_t k = wave; k * G + cu < n_units; k += CSW_THREADS / 64) {
        const uint32_t u = k * G + cu;                 // uniform
        const uint32_t p = u / nkh, kh = u % nkh;
        // p's token block: the lanes whose inclusive sum is at most p
        const uint32_t tb8 = (uint32_t) __builtin_popcountll(__ballot(inc <= p));
        const uint32_t before = tb8 > 0 ? __builtin_amdgcn_readlane(inc, tb8 - 1u) : 0u;
        chk_scores_unit(A, n_tok, kh / grp, kh % grp, tb8 * CSW_TOK, (p - before) * ATT_POS, lane);
    }
    // keep the read-ahead loads: their value goes nowhere (blockIdx.x never
    // equals gridDim.x)
    u32x4 x = ahead[0];
#pragma unroll
    for (int k = 1; k < AHEAD; ++k) x ^= ahead[k];
    if (blockIdx.x == gridDim.x) A.scores[0] = (float) (x[0] ^ x[1] ^ x[2] ^ x[3]);
}

// Softmax and p . V: workgroup (two query heads of a KV head, 8 head
// dimensions), eight waves.
//  - The softmax of each head's row (src/ops.c:386-422), on waves 4h ..
//    4h + 3: lane i of them holds the eight consecutive scores at 8i of each
//    span of 2048 positions; the max; ggml_v_expf over whole groups of eight, the C
//    library's expf over the rest (the tail group's wave, one term per
//    lane); the double sum with each group added as ((t0 + t1) + t2) + t3
//    of t_j = e_j + e_{j+4}, the groups in any order, checked, in the
//    reference's order when the check cannot decide; inv = 1/sum narrowed to
//    f32; p = e * inv. A head's waves meet in LDS for the max and for the
//    sum. For rows of at most 1536 positions the scores are loaded first,
//    one group per lane, and stay in registers. One wave issues a VALU
//    instruction every five or six cycles, so the exponentials of a row are
//    spread over the lanes, and a workgroup takes two query heads, not the
//    four of a KV head: the workgroups of one KV head share its slice of V
//    (they run on one XCD, where its L2 serves the repeat), not the
//    exponentials.
//  - The slice of V for the first 1536 positions is loaded by the two
//    producer waves, 3 and 7, 24 float4 per thread, once the scores are in.
//    In a row of at most 1536 positions those waves hold no scores: a wave
//    waits on its loads in the order it issued them, so a softmax wave with
//    V loads in flight would wait for them at its next use of a score.
//  - Per round of 1536 positions, p in LDS and the slice of V in the
//    producers' registers. In sub-rounds of 192 positions the producers form
//    the products p_s * v_s of every (head, dimension) into one of two LDS
//    buffers, while wave 0, one lane per (head, dimension), adds the previous sub-round's
//    products to its accumulator in order of s (src/forward.c:706-726) --
//    the chain wave issues adds and reads only.
__device__ __forceinline__ void pv_body(const dec_attn &A) {
    __shared__ __attribute__((aligned(16))) float P[PV_HPW][PV_RPOS];
    __shared__ __attribute__((aligned(16))) float X[2][PV_HPW * PV_SLICE][PV_XSTRIDE];
    __shared__ float stat_inv[PV_HPW], red_m[PV_WAVES];
    __shared__ double red_s[PV_WAVES];
    __shared__ uint64_t tab[32];          // the expf table, next to the lanes that index it
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t grp = A.n_head / A.n_kv, hd = A.hd, ss = A.sc_stride, slices = hd / PV_SLICE;
    const uint32_t wpk = (grp + PV_HPW - 1) / PV_HPW;      // workgroups per (KV head, slice)
    // workgroup -> (KV head, slice, its first query head). At most eight KV
    // heads: KV head h's workgroups all in column h of eight (XCD h, where
    // sllm_k_dec_scores left its scores and where its slices of V are read
    // twice), the other columns returning at once. Else the workgroups of
    // one (KV head, slice) on one XCD when the grid allows.
    uint32_t kvh, slice, j;
    {
        const uint32_t total = A.n_kv * slices * wpk, L = blockIdx.x;
        uint32_t p;
        if (A.n_kv <= 8) {
            if (L % 8u >= A.n_kv) return;
            const uint32_t r = L / 8u;
            p = (L % 8u) * slices + r / wpk;
            j = r % wpk;
        } else if (total % (8 * wpk) == 0) {
            const uint32_t per = total / 8, x = L % 8, r = L / 8;
            p = x * (per / wpk) + r / wpk;
            j = r % wpk;
        } else {
            p = L / wpk;
            j = L % wpk;
        }
        kvh = p / slices;
        slice = p % slices;
    }
    const uint32_t d0 = slice * PV_SLICE, qh0 = kvh * grp + j * PV_HPW;
    const uint32_t nh = min(PV_HPW, grp - j * PV_HPW);     // heads of this workgroup
    const uint32_t head = wave / PV_WPH, hw = wave % PV_WPH;
    const bool soft = head < nh;                          // uniform per wave
    const float *sc = A.scores + (size_t) (qh0 + min(head, nh - 1)) * ss;
    // this workgroup's slice of V: dimensions d0 .. d0 + 7 of every position, contiguous
    const float *vc = A.v_cache + ((size_t) kvh * A.n_ctx * hd + (size_t) slice * A.n_ctx * PV_SLICE);
    const uint32_t lpos = 8 * (hw * 64 + lane);         // the lane's first position in a span
    // eight scores from position s of the row (clamped inside the row: only
    // groups wholly past npast move)
    auto load8 = [&](uint32_t s, float (&v)[8]) {
        const uint32_t at = min(s, ss - 8);
        const f32x4 a = *G_CAST(const f32x4, sc + at), b = *G_CAST(const f32x4, sc + at + 4);
        v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
        v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
    };

    // (1) the loads that do not wait for the position, issued ahead of its
    // load: the lane's group of the first round (waves past it have none)
    // and the expf table
    const bool first_round_lane = soft && lpos < PV_RPOS;   // uniform per wave
    float sv[8];
    if (first_round_lane) load8(lpos, sv);
    const uint64_t tab_e = c_expf_tab[tid & 31u];
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t npast = (uint32_t) A.step->pos + 1;
    const uint32_t nb = npast / 8, nt = nb * 8;
    const bool one_round = npast <= PV_RPOS;
    // the tail group (positions nt .. npast - 1, if any): its span, wave of
    // the head's and lane
    const bool has_tail = npast > nt;
    const uint32_t t_span = nt / PV_SPAN, t_hw = (nt % PV_SPAN) / 512, t_lane = (nt % 512) / 8;

    auto group_sum = [](const float (&e)[8]) {
        const double t0 = (double) e[0] + (double) e[4], t1 = (double) e[1] + (double) e[5];
        const double t2 = (double) e[2] + (double) e[6], t3 = (double) e[3] + (double) e[7];
        return ((t0 + t1) + t2) + t3;
    };
    // e of the tail group (npast - nt <= 7 terms, the C library's expf),
    // held by lane lt: one term per lane, so that the wave evaluates expf
    // once rather than lane lt eight times over. Called by the whole wave.
    auto tail8 = [&](float (&v)[8], uint32_t lt, float m) {
        const uint32_t cnt = npast - nt;
        float xt = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float xi = lane_f(v[i], (int) lt);
            xt = lane == (uint32_t) i ? xi : xt;
        }
        float et = 0.0f;
        if (lane < cnt) et = sllm_libm_expf(xt - m, tab);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float ei = lane_f(et, i);
            if (lane == lt && (uint32_t) i < cnt) v[i] = ei;
        }
    };
    // e and the partial sum of the lane's group at s (whole groups through
    // ggml_v_expf; the tail group's terms already in v)
    auto exps_sum = [&](float (&v)[8], uint32_t s, float m, double &part) {
        if (s < nt) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = ggml_v_expf<true>(v[i] - m);
        }
        if (s + 8 <= npast) {
            part += group_sum(v);
        } else if (s < npast) {                       // the tail, from the lane's own registers
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (s + (uint32_t) i < npast) part += (double) v[i];
            }
        }
    };

    // producer pt holds float4 f = pt + 128 u of a round: position f / G4,
    // dimensions 4 (pt % G4) .. + 3 of the slice; its float4 3j .. 3j + 2
    // are sub-round j
    const bool producer = (wave & 3u) == 3;
    const uint32_t pt = (wave >> 2) * 64 + lane;
    f32x4 vr[PV_VLOADS];
    auto load_v = [&](uint32_t base) {
#pragma unroll
        for (int u = 0; u < PV_VLOADS; ++u) {
            const uint32_t f = pt + (uint32_t) u * PV_PTHREADS;
            const uint32_t sp = min(base + f / PV_G4, npast - 1);
            vr[u] = *G_CAST(const f32x4, vc + (size_t) sp * PV_SLICE + 4 * (f % PV_G4));
        }
    };

    // (2) the max of each head's row
    float m = -INFINITY;
    if (soft) {
        if (one_round) {
            if (first_round_lane) {
#pragma unroll
                for (int i = 0; i < 8; ++i) m = fmaxf(m, lpos + (uint32_t) i < npast ? sv[i] : -INFINITY);
            }
        } else {
            for (uint32_t b0 = 0; b0 < npast; b0 += PV_SPAN) {
                float v[8];
                const uint32_t s = b0 + lpos;
                load8(s, v);
#pragma unroll
                for (int i = 0; i < 8; ++i) m = fmaxf(m, s + (uint32_t) i < npast ? v[i] : -INFINITY);
            }
        }
    }
    m = wave_max(m);
    if (lane == 0) red_m[wave] = m;
    if (tid < 32) tab[tid] = tab_e;
    __syncthreads();                                 // red_m and the expf table visible

    // the producers' V (in a row of at most 1536 positions the producers
    // hold no scores)
    if (producer && one_round) load_v(0);

    // (3) e and the double sum of whole groups; the tail terms one lane each
    const uint32_t hb = min(head, PV_HPW - 1) * PV_WPH;  // the head's first wave
    m = red_m[hb];
#pragma unroll
    for (int w = 1; w < PV_WPH; ++w) m = fmaxf(m, red_m[hb + w]);
    double part = 0.0;
    if (soft) {
        if (one_round) {
            if (first_round_lane) {
                if (has_tail && t_hw == hw) tail8(sv, t_lane, m);     // uniform: the tail group's wave
                exps_sum(sv, lpos, m, part);
            }
        } else {
            for (uint32_t b0 = 0; b0 < npast; b0 += PV_SPAN) {
                float v[8];
                const uint32_t s = b0 + lpos;
                load8(s, v);
                if (has_tail && b0 == t_span * PV_SPAN && t_hw == hw) tail8(v, t_lane, m);   // uniform
                exps_sum(v, s, m, part);
                if (s < PV_RPOS) {                   // e of the first round, for p in place below
                    *reinterpret_cast<f32x4 *>(&P[head][s]) = (f32x4) { v[0], v[1], v[2], v[3] };
                    *reinterpret_cast<f32x4 *>(&P[head][s + 4]) = (f32x4) { v[4], v[5], v[6], v[7] };
                }
            }
        }
    }
    part = wave_sum_d(part);
    if (lane == 0) red_s[wave] = part;
    if (producer && !one_round) load_v(0);           // after this path's own score loads
    __syncthreads();                                 // red_s (and the first round's e) visible

    // (4) inv of each head, checked; p of the first round: from the e in
    // registers (one round), else in place over the e in LDS.
    // The reference's sum S lies within s (1 -+ b) of this order's s, b =
    // bound_f; its inv is (float) fl(1/S), and fl(1/S) lies within
    // r (1 -+ (b + 2^-50)) of r = fl(1/s). When both ends of that interval
    // narrow to one f32 -- the narrowing is monotone -- that f32 is the
    // reference's. One division per lane: lanes 32h .. 32h + 31 take head h.
    const double bound_f = (double) (nb + (npast - nt) + 8) * 0x1p-52;
    float inv_l;
    bool ok_l;
    {
        const uint32_t h = min(lane >> 5, PV_HPW - 1);
        double sum = red_s[h * PV_WPH];
#pragma unroll
        for (int w = 1; w < PV_WPH; ++w) sum += red_s[h * PV_WPH + w];
        const double r = 1.0 / sum, dr = r * (bound_f + 0x1p-50);
        inv_l = (float) (r - dr);
        ok_l = inv_l == (float) (r + dr) || h >= nh;
    }
    const bool ok_all = __builtin_amdgcn_readfirstlane((uint32_t) ok_l) != 0 &&
                        __builtin_amdgcn_readlane((uint32_t) ok_l, 32) != 0;    // uniform over the workgroup
    float inv = lane_f(inv_l, (int) (32 * min(head, PV_HPW - 1)));
    if (!ok_all) {
        // the reference's own order, one thread per head whose check cannot decide
        const bool mine = __builtin_amdgcn_readlane((uint32_t) ok_l, (int) (32 * min(head, PV_HPW - 1))) == 0;
        if (soft && mine && hw == 0 && lane == 0) {
            double seq = 0.0;
            for (uint32_t s = 0; s < nt; s += 8) {
                float v[8];
                load8(s, v);
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = ggml_v_expf<true>(v[i] - m);
                seq += group_sum(v);
            }
            for (uint32_t s = nt; s < npast; ++s) seq += (double) sllm_libm_expf(sc[s] - m, tab);
            stat_inv[head] = (float) (1.0 / seq);
        }
        __syncthreads();
        if (mine) inv = stat_inv[min(head, PV_HPW - 1)];
    }
    if (one_round) {
        if (first_round_lane && lpos < npast) {
            float *ph = &P[head][lpos];
            *reinterpret_cast<f32x4 *>(ph) = (f32x4) { sv[0] * inv, sv[1] * inv, sv[2] * inv, sv[3] * inv };
            *reinterpret_cast<f32x4 *>(ph + 4) = (f32x4) { sv[4] * inv, sv[5] * inv, sv[6] * inv, sv[7] * inv };
        }
    } else if (first_round_lane) {
#pragma unroll
        for (int i = 0; i < 8; i += 4) {
            f32x4 e4 = *reinterpret_cast<const f32x4 *>(&P[head][lpos + i]);
            e4[0] = e4[0] * inv; e4[1] = e4[1] * inv; e4[2] = e4[2] * inv; e4[3] = e4[3] * inv;
            *reinterpret_cast<f32x4 *>(&P[head][lpos + i]) = e4;
        }
    }

    // (5) rounds of 1536 positions, sub-rounds of 192
    const bool chain = wave == 0 && lane < nh * PV_SLICE;
    const uint32_t d4 = 4u * (pt % PV_G4);
    // products of sub-round j (positions 192 j ..) into X[buf]
    auto produce = [&](uint32_t j, int buf) {
        float pw[PV_VSUB][PV_HPW];                // every p read first, then the products
#pragma unroll
        for (int u = 0; u < PV_VSUB; ++u) {
            const uint32_t sl = (pt + (uint32_t) u * PV_PTHREADS) / PV_G4;
#pragma unroll
            for (int h = 0; h < (int) PV_HPW; ++h) pw[u][h] = P[h][PV_SUB * j + sl];
        }
#pragma unroll
        for (int u = 0; u < PV_VSUB; ++u) {
            const f32x4 v = vr[(int) (PV_VSUB * j) + u];     // j is a constant after unrolling
            const uint32_t sl = (pt + (uint32_t) u * PV_PTHREADS) / PV_G4;
#pragma unroll
            for (int h = 0; h < (int) PV_HPW; ++h) {
#pragma unroll
                for (int e = 0; e < 4; ++e) X[buf][(uint32_t) h * PV_SLICE + d4 + (uint32_t) e][sl] = pw[u][h] * v[e];
            }
        }
    };
    float acc = 0.0f;
    for (uint32_t base = 0; base < npast; base += PV_RPOS) {
        const uint32_t n = min(PV_RPOS, npast - base);
        if (base > 0) {
            __syncthreads();                      // the last round's products read
            if (producer) load_v(base);
            if (soft) {                           // p of this round, recomputed (the same bits)
                for (uint32_t i0 = 0; i0 < n; i0 += PV_SPAN) {
                    const uint32_t i = i0 + lpos;
                    float v[8];
                    load8(base + i, v);
                    const uint32_t r = nt - (base + i0);       // the tail group's offset in this pass
                    if (has_tail && r < PV_SPAN && r / 512 == hw) tail8(v, (r % 512) / 8, m);   // whole wave
                    if (base + i < nt) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) v[e] = ggml_v_expf<true>(v[e] - m);
                    }
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        if (i + (uint32_t) e < n) P[head][i + (uint32_t) e] = v[e] * inv;
                    }
                }
            }
        }
        __syncthreads();                          // this round's p in LDS
        const uint32_t n_sub = (n + PV_SUB - 1) / PV_SUB;
        if (producer) produce(0, 0);
        __syncthreads();
        // unrolled whole, so that the producers' register indices are constants
#pragma unroll
        for (uint32_t j = 0; j < PV_RPOS / PV_SUB; ++j) {
            if (j >= n_sub) break;                // uniform
            if (wave == 0) {
                if (chain) {
                    const float *x = X[j & 1u][lane];
                    const uint32_t cnt = min(PV_SUB, n - PV_SUB * j);
                    // sixteen products per block, three blocks in a ring: the
                    // reads for block s + 32 are in flight while block s is added
                    f32x4 qa[4], qb[4], qc[4];
                    auto rd = [&](uint32_t at, f32x4 (&q)[4]) {
                        const uint32_t c = min(at, PV_SUB - 16);
#pragma unroll
                        for (int t4 = 0; t4 < 4; ++t4) q[t4] = *reinterpret_cast<const f32x4 *>(x + c + 4 * t4);
                    };
                    auto add16 = [&](const f32x4 (&q)[4]) {
#pragma unroll
                        for (int t4 = 0; t4 < 4; ++t4) {
#pragma unroll
                            for (int e = 0; e < 4; ++e) acc = acc + q[t4][e];
                        }
                    };
                    uint32_t s = 0;
                    rd(0, qa);
                    rd(16, qb);
                    // (sched_barrier: the reads stay where they are issued, ahead
                    // of the adds they overlap)
                    for (; s + 48 <= cnt; s += 48) {
                        rd(s + 32, qc);
                        __builtin_amdgcn_sched_barrier(0);
                        add16(qa);
                        rd(s + 48, qa);
                        __builtin_amdgcn_sched_barrier(0);
                        add16(qb);
                        rd(s + 64, qb);
                        __builtin_amdgcn_sched_barrier(0);
                        add16(qc);
                    }
                    if (s + 16 <= cnt) {
                        add16(qa);
                        s += 16;
                        if (s + 16 <= cnt) {
                            add16(qb);
                            s += 16;
                        }
                    }
                    for (; s < cnt; ++s) acc = acc + x[s];
                }
            } else if (producer && j + 1 < n_sub) {
                produce(j + 1, (int) ((j + 1) & 1u));
            }
            __syncthreads();
        }
    }
    if (chain) A.out[(size_t) (qh0 + lane / PV_SLICE) * hd + d0 + lane % PV_SLICE] = acc;
}

extern "C" __global__ void __launch_bounds__(PV_THREADS)
sllm_k_dec_pv(dec_attn A) { pv_body(A); }

// ---------------------------------------------------------------------------
// output: x = a + b, RMSNorm with output_norm, the F16 rows
// (src/forward.c:800-827), then the argmax (src/forward.c:876-883) and the
// next token in a one-workgroup kernel
// ---------------------------------------------------------------------------

struct dec_lm {
    const float    *a, *b;       // the final residual is a + b
    const float    *norm_w;
    const uint16_t *embd;        // [n_vocab][n_embd] f16, the tied output projection
    float          *logits;
    uint64_t       *partial;     // one argmax key per workgroup
    dec_step       *step;
    float           eps;
    uint32_t        n_embd, n_vocab, pad;
};
static_assert(sizeof(dec_lm) == 72, "dec_lm must match decode.c");

constexpr int LM_THREADS = 256;
constexpr uint32_t LM_ROWS = 32;        // rows per pass: eight lanes per row
constexpr uint32_t LM_MAX_E = 8192;
constexpr int LM_UNROLL = 8;            // 64-element step pairs per load batch

// The argmax key of one logit: ordered like the float, -0 tied with +0, the
// lower row winning ties; NaN (never greater than anything) is 0.
__device__ __forceinline__ uint64_t argmax_key(float s, uint32_t row) {
    if (__builtin_isnan(s)) return 0;
    const uint32_t u = __float_as_uint(s == 0.0f ? 0.0f : s);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t) ord << 32) | (uint64_t) (0xffffffffu - row);
}

// Row . xn as src/ops.c:106-154 orders it: accumulator j (0..3) holds
// acc[j][0..7], element 32i + 8j + l going into acc[j][l] by FMA, i in
// order; then acc0 += acc2, acc1 += acc3, acc0 += acc1; t_l = acc0[l] +
// acc0[l+4]; (t0 + t1) + (t2 + t3). n_embd % 32 == 0, so there is no scalar
// tail. Eight lanes per row load its elements 64i' .. 64i' + 63 (steps 2i'
// and 2i' + 1): one load instruction is whole 128-byte runs of eight rows
// (sixteen rows x 64 bytes streams near 5 TB/s on MI355X against 6.9 for
// whole lines). Lane j < 4 holds accumulator j and takes step 2i''s eight
// elements from its own load and step 2i' + 1's from lane j + 4 (a DPP
// row shift), so each accumulator still sees its steps in order; lanes 4..7
// only load.
// Passes of 32 rows: workgroup w takes passes w, w + grid, w + 2 grid, ...;
// the host sizes the grid so that every workgroup has the same number of
// passes but the last few, which have one fewer (4008 passes over 501
// workgroups at 2B: eight each). Passes handed out by an atomic counter
// measured 1 % slower per token: the counter's atomics queue up. Each lane
// streams its rows in batches of eight 16-byte loads with the next batch
// always in flight, across a pass boundary too. The final residual and the
// norm weight are loaded before the first batch, so that the norm does not
// wait behind the weight stream (loads complete in order).
constexpr int LM_XV = (int) (LM_MAX_E / 4 / LM_THREADS);   // float4 of the residual per thread

extern "C" __global__ void __launch_bounds__(LM_THREADS)
sllm_k_dec_lm_head(dec_lm L) {
    __shared__ __attribute__((aligned(16))) float xn[LM_MAX_E];
    __shared__ double red_d[LM_THREADS / 64], lane_d[4];
    __shared__ uint64_t red_k[LM_THREADS / 64];
    const uint32_t e = L.n_embd, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t j = lane % 8, steps = e / 32, pairs = (steps + 1) / 2, nb = (pairs + LM_UNROLL - 1) / LM_UNROLL;
    const uint32_t n_pass = (L.n_vocab + LM_ROWS - 1) / LM_ROWS;

    // (1) the final residual and the norm weight, then the first batch
    f32x4 av[LM_XV], bv[LM_XV], wv[LM_XV];
#pragma unroll
    for (int u = 0; u < LM_XV; ++u) {
        const uint32_t i = min(4u * (tid + (uint32_t) u * LM_THREADS), e - 4);
        av[u] = *G_CAST(const f32x4, L.a + i);
        bv[u] = *G_CAST(const f32x4, L.b + i);
        wv[u] = *G_CAST(const f32x4, L.norm_w + i);
    }
    auto load = [&](uint32_t pass, uint32_t b, u32x4 (&h)[LM_UNROLL]) {
        const uint32_t row = min(pass * LM_ROWS + wave * 8 + lane / 8, L.n_vocab - 1);
        const GLOBAL u32x4 *w = G_CAST(const u32x4, L.embd + (size_t) row * e);
#pragma unroll
        for (int u = 0; u < LM_UNROLL; ++u) {
            const uint32_t pr = min(b * LM_UNROLL + u, pairs - 1);
            // an odd step past the row (n_embd % 64 == 32) reads the even one again
            const uint32_t jj = 2 * pr + j / 4 < steps ? j : j % 4;
            h[u] = __builtin_nontemporal_load(w + 8 * pr + jj);
        }
    };
    u32x4 ha[LM_UNROLL], hb[LM_UNROLL];
    uint32_t p = blockIdx.x;
    if (p < n_pass) load(p, 0, ha);

    // (2) RMSNorm of a + b into LDS
    double part = 0.0;
#pragma unroll
    for (int u = 0; u < LM_XV; ++u) {
        const uint32_t i = 4u * (tid + (uint32_t) u * LM_THREADS);
        if (i < e) {
            const f32x4 v = av[u] + bv[u];
            *reinterpret_cast<f32x4 *>(xn + i) = v;
#pragma unroll
            for (int c = 0; c < 4; ++c) part += (double) (v[c] * v[c]);
        }
    }
    const float mean = rms_mean(part, e, red_d, lane_d, [&](uint32_t k) { return L.a[k] + L.b[k]; });
    const float scale = 1.0f / sqrtf(mean + L.eps);
#pragma unroll
    for (int u = 0; u < LM_XV; ++u) {
        const uint32_t i = 4u * (tid + (uint32_t) u * LM_THREADS);
        if (i < e) {
            f32x4 x = *reinterpret_cast<const f32x4 *>(xn + i);
#pragma unroll
            for (int c = 0; c < 4; ++c) x[c] = (scale * x[c]) * wv[u][c];
            *reinterpret_cast<f32x4 *>(xn + i) = x;
        }
    }
    __syncthreads();                                        // xn complete
    uint32_t pn = p + gridDim.x;                            // the pass after p

    uint64_t best = 0;
    float acc[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
    auto consume = [&](uint32_t pass, uint32_t b, const u32x4 (&h)[LM_UNROLL]) {
#pragma unroll
        for (int u = 0; u < LM_UNROLL; ++u) {
            const uint32_t pr = b * LM_UNROLL + (uint32_t) u;
            if (pr < pairs) {                               // uniform
                const f32x8 hf = __builtin_convertvector(__builtin_bit_cast(f16x8, h[u]), f32x8);
                const float *x = xn + 64 * pr + 8 * (j % 4);
#pragma unroll
                for (int l = 0; l < 8; ++l) acc[l] = fmaf(hf[l], x[l], acc[l]);
                if (2 * pr + 1 < steps) {                   // uniform
#pragma unroll
                    for (int l = 0; l < 8; ++l) acc[l] = fmaf(dpp_mov_f<DPP_ROW_SHL4>(hf[l]), x[32 + l], acc[l]);
                }
            }
        }
        if (b == nb - 1) {                                // the row is complete
            float r[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) r[l] = acc[l] + dpp_mov_f<DPP_XOR2>(acc[l]);  // acc0 += acc2, acc1 += acc3
#pragma unroll
            for (int l = 0; l < 8; ++l) r[l] = r[l] + dpp_mov_f<DPP_XOR1>(r[l]);      // acc0 += acc1
            const float t0 = r[0] + r[4], t1 = r[1] + r[5], t2 = r[2] + r[6], t3 = r[3] + r[7];
            const float sdot = (t0 + t1) + (t2 + t3);
            const uint32_t row = pass * LM_ROWS + wave * 8 + lane / 8;
            if (j == 0 && row < L.n_vocab) {
                G_CAST(float, L.logits)[row] = sdot;
                const uint64_t key = argmax_key(sdot, row);
                best = key > best ? key : best;
            }
#pragma unroll
            for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
        }
    };
    // items (pass p, batch b) in order, the next one loaded before the
    // current one is used, buffers alternating by the item's parity
    uint32_t b = 0, it = 0;
    while (p < n_pass) {                                  // uniform
        uint32_t p2 = p, b2 = b + 1;
        if (b2 == nb) { p2 = pn; b2 = 0; }
        if (it & 1u) {
            if (p2 < n_pass) load(p2, b2, ha);
            consume(p, b, hb);
        } else {
            if (p2 < n_pass) load(p2, b2, hb);
            consume(p, b, ha);
        }
        ++it;
        p = p2;
        b = b2;
        if (b == 0) pn = p + gridDim.x;                   // entered pass p
    }

    best = wave_max_u64(best);
    if (lane == 0) red_k[wave] = best;
    __syncthreads();
    if (tid == 0) {
        uint64_t k = red_k[0];
        for (int i = 1; i < LM_THREADS / 64; ++i) k = red_k[i] > k ? red_k[i] : k;
        L.partial[blockIdx.x] = k;
    }
}

// The argmax over the output workgroups' keys (first maximum; a NaN first
// logit is never beaten, src/forward.c:876-883), and the step record moved
// on: next token from the prompt still to consume, else the argmax, which is
// also appended to the generated tokens.
extern "C" __global__ void __launch_bounds__(256)
sllm_k_dec_argmax(const uint64_t *__restrict__ partial, uint32_t n, const float *__restrict__ logits,
                  dec_step *__restrict__ st) {
    __shared__ uint64_t red[4];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    uint64_t best = 0;
    for (uint32_t i = tid; i < n; i += 256) best = partial[i] > best ? partial[i] : best;
    best = wave_max_u64(best);
    if (lane == 0) red[tid >> 6] = best;
    __syncthreads();
    if (tid != 0) return;
    for (int i = 1; i < 4; ++i) best = red[i] > best ? red[i] : best;
    int32_t next = best == 0 ? 0 : (int32_t) (0xffffffffu - (uint32_t) best);
    if (__builtin_isnan(logits[0])) next = 0;
    st->next = next;
    if (st->advance) {
        if (st->i_feed < st->n_feed) {
            st->token = st->feed[st->i_feed];
            st->i_feed += 1;
        } else {
            if (st->gen != nullptr && st->n_gen < st->cap_gen) st->gen[st->n_gen] = next;
            st->n_gen += 1;
            st->token = next;
        }
        st->pos += 1;
    }
}

// ---------------------------------------------------------------------------
// chunks of tokens (src/forward.c:589-835 with n > 1): per-token kernels
// around the batched MFMA GEMM (i2s_kernels.hip), the chunk modes of the
// attention kernels above, and the output head over every token
// ---------------------------------------------------------------------------

namespace {

enum : uint32_t { IN_SILU = 3 };

// One token's activation, built, normalised and quantised: row t of a
// [n][k] layout per workgroup.
struct chk_prep {
    const void    *a;          // IN_EMBED: f16 rows [n_vocab][k]; else f32 [n][k] (IN_SILU: gate)
    const float   *b;          // IN_RESID: added to a; IN_SILU: up
    const int32_t *tokens;     // IN_EMBED: the chunk's tokens
    float         *v_out;      // the vector as built, [n][k], or null
    const float   *norm_w;     // RMSNorm weight, k floats
    int8_t        *q_out;      // the quantised rows [n][k], or null
    act_t         *act_out;    // their scale / sum [n], or null
    float         *xn_out;     // the normalised rows [n][k] (the output head's input), or null
    float          eps;
    uint32_t       k, mode, pad;
};
static_assert(sizeof(chk_prep) == 80, "chk_prep must match decode.c");

constexpr int CHK_THREADS = 512;        // eight waves per token (measured: four leave the SIMDs half idle)
constexpr uint32_t CHK_MAX_K = 7168;

// The output head over a chunk: logits[t][r] = row r . xn[t] for every
// token (src/forward.c:800-827 with n > 1).
struct chk_lm {
    const float    *xn;        // [n][n_embd]
    const uint16_t *embd;      // [n_vocab][n_embd] f16
    float          *logits;    // [n][n_vocab]
    uint32_t        n_embd, n_vocab, n_tok, n_wg;
};
static_assert(sizeof(chk_lm) == 40, "chk_lm must match decode.c");

constexpr int CLM_THREADS = 256;        // one row per lane
constexpr int CLM_TOK = 4;              // tokens per workgroup

} // namespace

// Workgroup t: token t's vector (the embedding lookup; a residual sum;
// silu(gate) * up as src/forward.c:776-778), kept in v_out if asked; RMSNorm
// (src/ops.c:254-322) with the same mean as the decode step's; then either
// the normalised row (xn_out) or its quantisation (src/i2s_gemm.c:45-83).
// One straight path per input mode and width (CU float4 per thread): every
// input load is unconditional (addresses clamped inside the row) and goes
// out before the first is used, so the loads overlap instead of each waiting
// behind the last one's stores.
template <uint32_t MODE, int CU, int TH>
__device__ __forceinline__ void chk_prep_body(const chk_prep &P, float *xs, double *red_d, double *lane_d,
                                              float *red_f, int *red_i) {
    const uint32_t t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, k = P.k;
    const size_t row = (size_t) t * k;
    const int32_t token = MODE == IN_EMBED ? P.tokens[t] : 0;
    f32x4 va[CU], vb[CU], wv[CU];
    u32x2 ha[CU];
#pragma unroll
    for (int u = 0; u < CU; ++u) {
        const uint32_t i = min(4 * tid + 4 * TH * (uint32_t) u, k - 4);
        if (MODE == IN_EMBED) {
            ha[u] = *G_CAST(const u32x2, (const uint16_t *) P.a + (size_t) token * k + i);
        } else {
            va[u] = *G_CAST(const f32x4, (const float *) P.a + row + i);
            if (MODE != IN_PLAIN) vb[u] = *G_CAST(const f32x4, P.b + row + i);
        }
        // the norm weights beside the vector rather than after the mean
        wv[u] = *G_CAST(const f32x4, P.norm_w + i);
    }
    double part = 0.0;
#pragma unroll
    for (int u = 0; u < CU; ++u) {
        const uint32_t i = 4 * tid + 4 * TH * (uint32_t) u;
        if (i < k) {
            f32x4 v;
            if (MODE == IN_EMBED) {
                v = (f32x4) { embd_f32(ha[u][0] & 0xffffu), embd_f32(ha[u][0] >> 16), embd_f32(ha[u][1] & 0xffffu),
                              embd_f32(ha[u][1] >> 16) };
            } else if (MODE == IN_RESID) {
                v = va[u] + vb[u];
            } else if (MODE == IN_SILU) {
#pragma unroll
                for (int c = 0; c < 4; ++c) v[c] = silu(va[u][c]) * vb[u][c];
            } else {
                v = va[u];
            }
            *reinterpret_cast<f32x4 *>(xs + i) = v;
            if (P.v_out != nullptr) *G_CAST(f32x4, P.v_out + row + i) = v;
#pragma unroll
            for (int c = 0; c < 4; ++c) part += (double) (v[c] * v[c]);
        }
    }
    const float mean = rms_mean(part, k, red_d, lane_d, [&](uint32_t j) { return xs[j]; });
    const float scale = 1.0f / sqrtf(mean + P.eps);
    float m = 0.0f;
#pragma unroll
    for (int u = 0; u < CU; ++u) {
        const uint32_t i = 4 * tid + 4 * TH * (uint32_t) u;
        if (i < k) {
            f32x4 v = *reinterpret_cast<const f32x4 *>(xs + i);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                v[c] = (scale * v[c]) * wv[u][c];
                m = fmaxf(m, fabsf(v[c]));
            }
            *reinterpret_cast<f32x4 *>(xs + i) = v;
            if (P.xn_out != nullptr) *G_CAST(f32x4, P.xn_out + row + i) = v;
        }
    }
    if (P.q_out == nullptr) return;                  // uniform
    m = wave_max(m);
    if (lane == 0) red_f[wave] = m;
    __syncthreads();
    m = red_f[0];
#pragma unroll
    for (int w = 1; w < TH / 64; ++w) m = fmaxf(m, red_f[w]);
    const float qs = m > 0.0f ? 127.0f / m : 0.0f;
    int ls = 0;
#pragma unroll
    for (int u = 0; u < CU; ++u) {
        const uint32_t i = 4 * tid + 4 * TH * (uint32_t) u;
        if (i < k) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(xs + i);
            const int a = quant_one(v[0] * qs), b = quant_one(v[1] * qs);
            const int c = quant_one(v[2] * qs), e = quant_one(v[3] * qs);
            ls += a + b + c + e;
            *G_CAST(uint32_t, P.q_out + row + i) =
                (uint32_t) (a & 0xff) | ((uint32_t) (b & 0xff) << 8) | ((uint32_t) (c & 0xff) << 16) |
                ((uint32_t) (e & 0xff) << 24);
        }
    }
    ls = wave_sum(ls);
    if (lane == 0) red_i[wave] = ls;
    __syncthreads();
    if (tid == 0) {
        int32_t asum = 0;
#pragma unroll
        for (int w = 0; w < TH / 64; ++w) asum += red_i[w];
        G_CAST(float, P.act_out + t)[0] = qs;
        G_CAST(int32_t, P.act_out + t)[1] = asum;
    }
}

template <int CU, int TH>
__device__ __forceinline__ void chk_prep_width(const chk_prep &P, float *xs, double *red_d, double *lane_d,
                                               float *red_f, int *red_i) {
    switch (P.mode) {
    case IN_EMBED: chk_prep_body<IN_EMBED, CU, TH>(P, xs, red_d, lane_d, red_f, red_i); break;
    case IN_RESID: chk_prep_body<IN_RESID, CU, TH>(P, xs, red_d, lane_d, red_f, red_i); break;
    case IN_SILU:  chk_prep_body<IN_SILU, CU, TH>(P, xs, red_d, lane_d, red_f, red_i); break;
    default:       chk_prep_body<IN_PLAIN, CU, TH>(P, xs, red_d, lane_d, red_f, red_i); break;
    }
}

template <int TH>
__device__ __forceinline__ void chk_prep_entry(const chk_prep &P) {
    __shared__ __attribute__((aligned(16))) float xs[CHK_MAX_K];
    __shared__ double red_d[TH / 64], lane_d[4];
    __shared__ float red_f[TH / 64];
    __shared__ int red_i[TH / 64];
    constexpr int CU_S = (3072 + 4 * TH - 1) / (4 * TH);    // widths up to 3072 (n_embd), then up to CHK_MAX_K
    if (P.k <= 4u * TH * CU_S) chk_prep_width<CU_S, TH>(P, xs, red_d, lane_d, red_f, red_i);
    else chk_prep_width<(int) ((CHK_MAX_K + 4 * TH - 1) / (4 * TH)), TH>(P, xs, red_d, lane_d, red_f, red_i);
}

extern "C" __global__ void __launch_bounds__(CHK_THREADS)
sllm_k_chk_prep(chk_prep P) { chk_prep_entry<CHK_THREADS>(P); }

// Workgroup t: token t's key roped at its position (NeoX, src/ops.c:467-549)
// and stored with its value into the caches (src/forward.c:668-690), so that
// every query of the chunk finds the keys at or before its position; and the
// token's queries roped in place, so that the scores read them as they are.
// The query and key rows and the position's cos / sin are read into LDS
// first, in one round of loads (each output needs its pair's input).
constexpr uint32_t KVS_MAX_Q = 7168;    // a query row: n_head * hd <= the decoder's widest row

extern "C" __global__ void __launch_bounds__(ATT_THREADS)
sllm_k_chk_kv_store(dec_attn A) {
    __shared__ float qs[KVS_MAX_Q], ks[KVS_MAX_Q], cst[ATT_MAX_HD];
    const uint32_t t = blockIdx.x, pos = A.chunk_base + t, hd = A.hd, half = A.half;
    const uint32_t gqa = A.n_kv * hd, nq = A.n_head * hd;
    const float *cs = A.rope + (size_t) pos * (half > 0 ? half : 1) * 2;
    const float *k = A.k + (size_t) t * gqa, *v = A.v + (size_t) t * gqa;
    float *q = const_cast<float *>(A.q) + (size_t) t * nq;
    for (uint32_t i = threadIdx.x; i < nq; i += ATT_THREADS) qs[i] = q[i];
    for (uint32_t i = threadIdx.x; i < gqa; i += ATT_THREADS) {
        ks[i] = k[i];
        // values slice-major: [KV head][dimension / 8][position][dimension % 8]
        A.v_cache[(((size_t) (i / hd) * (hd / PV_SLICE) + (i % hd) / PV_SLICE) * A.n_ctx + pos) * PV_SLICE +
                  i % PV_SLICE] = v[i];
    }
    for (uint32_t i = threadIdx.x; i < 2 * half; i += ATT_THREADS) cst[i] = cs[i];
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < gqa; i += ATT_THREADS) {
        const uint32_t kvh = i / hd, d = i % hd;
        const rope_in r = rope_load(ks + (size_t) kvh * hd, d, half, cst);
        A.k_cache[(((size_t) kvh * (hd / PV_SLICE) + d / PV_SLICE) * A.n_ctx + pos) * PV_SLICE + d % PV_SLICE] =
            rope_apply(r, d, half);
    }
    for (uint32_t i = threadIdx.x; i < nq; i += ATT_THREADS) {
        const uint32_t hh = i / hd, d = i % hd;
        const rope_in r = rope_load(qs + (size_t) hh * hd, d, half, cst);
        q[i] = rope_apply(r, d, half);
    }
}

// The output head over a chunk. Lane = one row; a workgroup takes 256 rows
// for CLM_TOK tokens. Each row . xn[t] is formed as src/ops.c:106-154 orders
// it: accumulator 8j + l collects element 32i + 8j + l by FMA over i; then
// (acc_0 + acc_2) + (acc_1 + acc_3) per l, t_l = a_l + a_{l+4},
// (t0 + t1) + (t2 + t3). The normalised rows are the same for every lane,
// so they are read as wave-uniform values. Workgroups for the same rows sit
// next to each other on one XCD, so the rows come from its L2 after the
// first token block.
extern "C" __global__ void __launch_bounds__(CLM_THREADS)
sllm_k_chk_lm_head(chk_lm L) {
    const uint32_t n_tb = (L.n_tok + CLM_TOK - 1) / CLM_TOK;
    const uint32_t b = xcd_slot(L.n_wg);
    const uint32_t tb = b % n_tb, rb = b / n_tb;
    const uint32_t e = L.n_embd, steps = e / 32;
    if (rb * CLM_THREADS >= L.n_vocab) return;
    const uint32_t row = min(rb * CLM_THREADS + threadIdx.x, L.n_vocab - 1);
    const uint32_t t0 = tb * CLM_TOK;
    const GLOBAL u32x4 *w = G_CAST(const u32x4, L.embd + (size_t) row * e);
    // the normalised rows do not change during the launch: constant
    // address space, so the wave-uniform reads are scalar loads
    typedef __attribute__((address_space(4))) const float cfloat;
    cfloat *xb[CLM_TOK];
#pragma unroll
    for (int u = 0; u < CLM_TOK; ++u) xb[u] = (cfloat *) (L.xn + (size_t) min(t0 + (uint32_t) u, L.n_tok - 1) * e);
    float acc[CLM_TOK][32];
#pragma unroll
    for (int u = 0; u < CLM_TOK; ++u) {
#pragma unroll
        for (int j = 0; j < 32; ++j) acc[u][j] = 0.0f;
    }
    // 32 elements (64 bytes) of the row per step; steps alternate between
    // two buffers so that the next step's loads are in flight during this one
    auto load = [&](uint32_t i, u32x4 (&h)[4]) {
        const uint32_t at = 4 * min(i, steps - 1);
#pragma unroll
        for (int c = 0; c < 4; ++c) h[c] = w[at + (uint32_t) c];
    };
    auto step = [&](uint32_t i, const u32x4 (&h)[4]) {
        float hf[32];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const f32x8 f = __builtin_convertvector(__builtin_bit_cast(f16x8, h[c]), f32x8);
#pragma unroll
            for (int l = 0; l < 8; ++l) hf[8 * c + l] = f[l];
        }
#pragma unroll
        for (int u = 0; u < CLM_TOK; ++u) {
            cfloat *x = xb[u] + 32 * i;
#pragma unroll
            for (int j = 0; j < 32; ++j) acc[u][j] = fmaf(hf[j], x[j], acc[u][j]);
        }
    };
    u32x4 ha[4], hb[4];
    load(0, ha);
    uint32_t i = 0;
    for (; i + 1 < steps; i += 2) {
        load(i + 1, hb);
        step(i, ha);
        load(i + 2, ha);
        step(i + 1, hb);
    }
    if (i < steps) step(i, ha);
    if (rb * CLM_THREADS + threadIdx.x >= L.n_vocab) return;
#pragma unroll
    for (int u = 0; u < CLM_TOK; ++u) {
        if (t0 + (uint32_t) u < L.n_tok) {
            float a[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) a[l] = (acc[u][l] + acc[u][16 + l]) + (acc[u][8 + l] + acc[u][24 + l]);
            const float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
            L.logits[(size_t) (t0 + (uint32_t) u) * L.n_vocab + row] = (s0 + s1) + (s2 + s3);
        }
    }
}

// The chunk's softmax rows: one wave per (token, query head) row, or half
// a wave for rows of at most 256 positions; the decode step's operations
// (src/ops.c:386-422) -- the max; ggml_v_expf over
// whole groups of eight, the C library's expf over the rest; the double sum
// of the groups (((e0+e4) + (e1+e5)) + (e2+e6)) + (e3+e7) and of the tail
// terms in any order, checked, in the reference's order when the check
// cannot decide; inv = 1/sum -- then p_s = e_s * inv written back over the
// row for s < npast (e recomputed for rows past 512 positions: the same
// bits).
constexpr int CSM_THREADS = 256;        // four waves per workgroup

// One row of at most 512 positions or more, a whole wave (lane l holds
// positions 8l .. 8l + 7 of each block of 512)
__device__ __forceinline__ void csm_full_row(const dec_attn &A, uint32_t row_i, uint32_t lane, const uint64_t *tab) {
    const uint32_t t = row_i / A.n_head, hh = row_i % A.n_head, ss = A.sc_stride;
    const uint32_t npast = A.chunk_base + t + 1, nb = npast / 8, nt = nb * 8;
    float *sc = A.scores + (size_t) t * A.n_head * ss + (size_t) hh * ss;

    auto group_sum = [](const float (&e)[8]) {
        const double t0 = (double) e[0] + (double) e[4], t1 = (double) e[1] + (double) e[5];
        const double t2 = (double) e[2] + (double) e[6], t3 = (double) e[3] + (double) e[7];
        return ((t0 + t1) + t2) + t3;
    };
    auto load8 = [&](uint32_t s, float (&v)[8]) {
        const uint32_t at = min(s, ss - 8);
        const f32x4 a = *G_CAST(const f32x4, sc + at), b = *G_CAST(const f32x4, sc + at + 4);
        v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
        v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
    };
    auto store8 = [&](uint32_t s, const float (&v)[8], float inv) {
        *G_CAST(f32x4, sc + s) = (f32x4) { v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv };
        *G_CAST(f32x4, sc + s + 4) = (f32x4) { v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv };
    };
    auto exps8 = [&](float (&v)[8], uint32_t s, float m) {
        if (s < nt) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = ggml_v_expf<true>(v[i] - m);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = sllm_libm_expf(v[i] - m, tab);
        }
    };
    // e of whole groups (lanes whose group lies below nt)
    auto ggml8 = [&](float (&v)[8], uint32_t s, float m) {
        if (s < nt) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = ggml_v_expf<true>(v[i] - m);
        }
    };
    // e of the tail group (npast - nt <= 7 terms, the C library's expf),
    // held by lane lt: one term per lane, so that the wave evaluates expf
    // once rather than lane lt eight times over. Called by the whole wave.
    auto tail8 = [&](float (&v)[8], uint32_t lt, float m) {
        const uint32_t cnt = npast - nt;
        float xt = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float xi = lane_f(v[i], (int) lt);
            xt = lane == (uint32_t) i ? xi : xt;
        }
        float et = 0.0f;
        if (lane < cnt) et = sllm_libm_expf(xt - m, tab);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float ei = lane_f(et, i);
            if (lane == lt && (uint32_t) i < cnt) v[i] = ei;
        }
    };
    const bool has_tail = npast > nt;
    auto add_group = [&](double &part, const float (&v)[8], uint32_t s) {
        if (s + 8 <= npast) {
            part += group_sum(v);
        } else {                                   // the tail, term by term
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (s + (uint32_t) i < npast) part += (double) v[i];
            }
        }
    };

    float m = -INFINITY;
    double part = 0.0;
    float v1[8];                                    // a row of one round stays in registers
    if (npast <= 512) {
        const uint32_t s = 8 * lane;
        load8(s, v1);
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, s + (uint32_t) i < npast ? v1[i] : -INFINITY);
        m = wave_max(m);
        if (has_tail) tail8(v1, nt / 8u, m);
        if (s < npast) {
            ggml8(v1, s, m);
            add_group(part, v1, s);
        }
    } else {
        for (uint32_t b0 = 0; b0 < npast; b0 += 512) {
            float v[8];
            const uint32_t s = b0 + 8 * lane;
            load8(s, v);
#pragma unroll
            for (int i = 0; i < 8; ++i) m = fmaxf(m, s + (uint32_t) i < npast ? v[i] : -INFINITY);
        }
        m = wave_max(m);
        for (uint32_t b0 = 0; b0 < npast; b0 += 512) {
            float v[8];
            const uint32_t s = b0 + 8 * lane;
            load8(s, v);
            if (has_tail && nt - b0 < 512u) tail8(v, (nt - b0) / 8u, m);   // uniform
            if (s < npast) {
                ggml8(v, s, m);
                add_group(part, v, s);
            }
        }
    }
    // inv = 1/sum from the lanes' partial sums: checked, else the reference's
    // order by one lane
    const double sum = wave_sum_d(part);
    const double bound = sum * ((double) (nb + (npast - nt) + 8) * 0x1p-52);
    float inv = (float) (1.0 / (sum - bound));
    if (inv != (float) (1.0 / (sum + bound))) {     // uniform over the wave
        if (lane == 0) {
            double seq = 0.0;
            for (uint32_t s = 0; s < nt; s += 8) {
                float v[8];
                load8(s, v);
                exps8(v, s, m);
                seq += group_sum(v);
            }
            for (uint32_t s = nt; s < npast; ++s) seq += (double) sllm_libm_expf(sc[s] - m, tab);
            inv = (float) (1.0 / seq);
        }
        inv = lane_f(inv, 0);
    }
    // every lane's reads of the row are done (the wave reduced them above)
    if (npast <= 512) {
        const uint32_t s = 8 * lane;
        if (s < npast) store8(s, v1, inv);
    } else {
        for (uint32_t b0 = 0; b0 < npast; b0 += 512) {
            float v[8];
            const uint32_t s = b0 + 8 * lane;
            load8(s, v);
            if (has_tail && nt - b0 < 512u) tail8(v, (nt - b0) / 8u, m);   // uniform
            if (s < npast) {
                ggml8(v, s, m);
                store8(s, v, inv);
            }
        }
    }
}
// The max and the double sum over the 32 lanes of each half of the wave
// (every lane gets its half's), as wave_max / wave_sum_d
__device__ __forceinline__ float half_max(float v) {
    v = fmaxf(v, dpp_mov_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_mov_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_mov_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_mov_f<DPP_MIRROR>(v));
    const float lo = fmaxf(lane_f(v, 0), lane_f(v, 16)), hi = fmaxf(lane_f(v, 32), lane_f(v, 48));
    return (threadIdx.x & 32u) ? hi : lo;
}

__device__ __forceinline__ double half_sum_d(double v) {
    v += dpp_mov_d<DPP_XOR1>(v);
    v += dpp_mov_d<DPP_XOR2>(v);
    v += dpp_mov_d<DPP_HALF_MIRROR>(v);
    v += dpp_mov_d<DPP_MIRROR>(v);
    const double lo = read_lane_d(v, 0) + read_lane_d(v, 16), hi = read_lane_d(v, 32) + read_lane_d(v, 48);
    return (threadIdx.x & 32u) ? hi : lo;
}

// Rows of at most 256 positions, two to a wave: lanes 0..31 take row ra,
// lanes 32..63 row rb (lane 32h + j holds positions 8j .. 8j + 7), each half
// with the operations of csm_full_row over its own lanes. two = false: rb
// repeats ra and its half stores nothing.
constexpr uint32_t CSM_HALF = 256;

__device__ __forceinline__ void csm_pair_rows(const dec_attn &A, uint32_t ra, uint32_t rb, bool two, uint32_t lane,
                                              const uint64_t *tab) {
    const uint32_t hw = lane >> 5, lh = lane & 31u, ss = A.sc_stride;
    const uint32_t r = hw ? rb : ra;
    const uint32_t t = r / A.n_head, hh = r % A.n_head;
    const uint32_t npast = A.chunk_base + t + 1, nb = npast / 8, nt = nb * 8;
    float *sc = A.scores + (size_t) t * A.n_head * ss + (size_t) hh * ss;
    // each row's tail group (its lane within the half), for wave-uniform lane reads
    const uint32_t lta = min((A.chunk_base + ra / A.n_head + 1) / 8u, 31u);
    const uint32_t ltb = min((A.chunk_base + rb / A.n_head + 1) / 8u, 31u);

    auto group_sum = [](const float (&e)[8]) {
        const double t0 = (double) e[0] + (double) e[4], t1 = (double) e[1] + (double) e[5];
        const double t2 = (double) e[2] + (double) e[6], t3 = (double) e[3] + (double) e[7];
        return ((t0 + t1) + t2) + t3;
    };
    auto load8 = [&](uint32_t s, float (&v)[8]) {
        const uint32_t at = min(s, ss - 8);
        const f32x4 a = *G_CAST(const f32x4, sc + at), b = *G_CAST(const f32x4, sc + at + 4);
        v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
        v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
    };

    const uint32_t s = 8 * lh;
    float v[8];
    load8(s, v);
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, s + (uint32_t) i < npast ? v[i] : -INFINITY);
    m = half_max(m);
    // the tail group (npast - nt <= 7 terms, the C library's expf): term i of
    // each half's tail evaluated by lane i of that half
    {
        const uint32_t cnt = npast - nt, lt = nt / 8u;
        float xt = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float xa = lane_f(v[i], (int) lta), xb = lane_f(v[i], 32 + (int) ltb);
            xt = lh == (uint32_t) i ? (hw ? xb : xa) : xt;
        }
        float et = 0.0f;
        if (lh < cnt) et = sllm_libm_expf(xt - m, tab);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float ea = lane_f(et, i), eb = lane_f(et, 32 + i);
            if (lh == lt && (uint32_t) i < cnt) v[i] = hw ? eb : ea;
        }
    }
    double part = 0.0;
    if (s < nt) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = ggml_v_expf<true>(v[i] - m);
        part = group_sum(v);
    } else if (s < npast) {                        // the tail, term by term
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (s + (uint32_t) i < npast) part += (double) v[i];
        }
    }
    // inv = 1/sum: checked, else the reference's order by the half's first lane
    const double sum = half_sum_d(part);
    const double bound = sum * ((double) (nb + (npast - nt) + 8) * 0x1p-52);
    float inv = (float) (1.0 / (sum - bound));
    if (inv != (float) (1.0 / (sum + bound))) {     // uniform over the half
        if (lh == 0) {
            double seq = 0.0;
            for (uint32_t q = 0; q < nt; q += 8) {
                float e[8];
                load8(q, e);
#pragma unroll
                for (int i = 0; i < 8; ++i) e[i] = ggml_v_expf<true>(e[i] - m);
                seq += group_sum(e);
            }
            for (uint32_t q = nt; q < npast; ++q) seq += (double) sllm_libm_expf(sc[q] - m, tab);
            inv = (float) (1.0 / seq);
        }
    }
    {
        const float ia = lane_f(inv, 0), ib = lane_f(inv, 32);
        inv = hw ? ib : ia;
    }
    if (s < npast && (two || hw == 0)) {
        *G_CAST(f32x4, sc + s) = (f32x4) { v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv };
        *G_CAST(f32x4, sc + s + 4) = (f32x4) { v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv };
    }
}

// The rows of tokens whose npast is at most CSM_HALF come first, two to a
// wave, then one row per wave; the host sizes the grid with the same count
// (csm_waves).
__device__ __forceinline__ uint32_t csm_short_rows(const dec_attn &A, uint32_t n_tok) {
    return (A.chunk_base >= CSM_HALF ? 0u : min(CSM_HALF - A.chunk_base, n_tok)) * A.n_head;
}

extern "C" __global__ void __launch_bounds__(CSM_THREADS)
sllm_k_chk_softmax(dec_attn A, uint32_t n_tok) {
    __shared__ uint64_t tab[32];
    if (threadIdx.x < 32) tab[threadIdx.x] = c_expf_tab[threadIdx.x];
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t w = blockIdx.x * (CSM_THREADS / 64) + wave;
    const uint32_t n_short = csm_short_rows(A, n_tok), w_short = (n_short + 1) / 2;
    if (w < w_short) {                              // uniform
        const bool two = 2 * w + 1 < n_short;
        csm_pair_rows(A, 2 * w, two ? 2 * w + 1 : 2 * w, two, lane, tab);
        return;
    }
    const uint32_t row_i = n_short + (w - w_short);
    if (row_i >= n_tok * A.n_head) return;          // uniform
    csm_full_row(A, row_i, lane, tab);
}

// The chunk's p . V in units of one wave: (KV head, query head h, half of
// the head dimensions, 4 tokens), one dimension per lane. Each lane adds
// p_s * v_s to four chains -- its dimension for the four tokens -- in order
// of s (src/forward.c:706-726), a token's chain left alone past its own
// position. p (written over the scores rows by sllm_k_chk_softmax) is the
// same for every lane of a wave and comes through the scalar unit, eight
// positions of a token per load; V rows stream from L2 two blocks of
// sixteen positions ahead.
constexpr uint32_t CP_TOK = 4;
constexpr int CP_THREADS = 1024;

__device__ __forceinline__ void chk_pv_unit(const dec_attn &A, uint32_t n_tok, uint32_t kvh, uint32_t tb,
                                            uint32_t lane, uint32_t h, uint32_t half_id) {
    const uint32_t grp = A.n_head / A.n_kv, hd = A.hd, ss = A.sc_stride;
    const uint32_t last_tok = min(tb + CP_TOK, n_tok) - 1;
    const uint32_t npast_max = A.chunk_base + last_tok + 1, npast_min = A.chunk_base + tb + 1;
    const uint32_t d = min(64u * half_id + lane, hd - 1);
    // dimension d of position s: slice d / 8, element d % 8
    const float *vc = A.v_cache + ((size_t) kvh * (hd / PV_SLICE) + d / PV_SLICE) * A.n_ctx * PV_SLICE + d % PV_SLICE;
    // p is not written during the launch: constant address space, so that
    // its wave-uniform reads are scalar loads
    typedef __attribute__((address_space(4))) const f32x8 cf32x8;
    typedef __attribute__((address_space(4))) const float cfloat;
    cfloat *prow[CP_TOK];                          // token rows past n_tok read the last one's
    float acc[CP_TOK];
    uint32_t npast_t[CP_TOK];                      // each token's own (past n_tok: never written out)
#pragma unroll
    for (int tk = 0; tk < (int) CP_TOK; ++tk) {
        prow[tk] = (cfloat *) (A.scores + ((size_t) min(tb + (uint32_t) tk, last_tok) * A.n_head + kvh * grp + h) * ss);
        acc[tk] = 0.0f;
        npast_t[tk] = A.chunk_base + tb + (uint32_t) tk + 1;
    }
    // p of positions s..s+7 of token tk (within the row: sc_stride >= n_ctx, a multiple of 8)
    auto p8 = [&](int tk, uint32_t s) { return *(cf32x8 *) (prow[tk] + min(s, ss - 8)); };
    float va[16], vb[16];
    auto load16 = [&](uint32_t s, float (&v)[16]) {
#pragma unroll
        for (int q = 0; q < 16; ++q) v[q] = *G_CAST(const float, vc + (size_t) min(s + (uint32_t) q, npast_max - 1) * PV_SLICE);
    };
    // eight positions at which every token of the block is live, with p of
    // them in pc; the next eight's p go to pn. Scalar loads return out of
    // order, so a wait covers all of them: the next loads are issued only
    // after the first use of pc has waited for it.
    auto step8 = [&](uint32_t s, const float *v, const f32x8 (&pc)[CP_TOK], f32x8 (&pn)[CP_TOK]) {
#pragma unroll
        for (int tk = 0; tk < (int) CP_TOK; ++tk) acc[tk] = acc[tk] + pc[tk][0] * v[0];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int tk = 0; tk < (int) CP_TOK; ++tk) pn[tk] = p8(tk, s + 8);
        __builtin_amdgcn_sched_barrier(0);
        // per position the four products, then the four sums: no sum right
        // behind the product it waits for (a wave alone on its SIMD)
#pragma unroll
        for (int q = 1; q < 8; ++q) {
            float x[CP_TOK];
#pragma unroll
            for (int tk = 0; tk < (int) CP_TOK; ++tk) x[tk] = pc[tk][q] * v[q];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int tk = 0; tk < (int) CP_TOK; ++tk) acc[tk] = acc[tk] + x[tk];
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    f32x8 pa[CP_TOK], pb[CP_TOK];
#pragma unroll
    for (int tk = 0; tk < (int) CP_TOK; ++tk) pa[tk] = p8(tk, 0);
    // sixteen positions: p of the first eight in pa on entry, of the next
    // sixteen's first eight in pa on exit
    auto step16 = [&](uint32_t s, const float (&v)[16]) {
        step8(s, v, pa, pb);
        step8(s + 8, v + 8, pb, pa);
    };
    // the last positions: a token's chain left alone past its own
    auto tail = [&](uint32_t s, uint32_t r, const float (&v)[16]) {
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            if (8u * (uint32_t) hb < r) {
                f32x8 p[CP_TOK];
#pragma unroll
                for (int tk = 0; tk < (int) CP_TOK; ++tk) p[tk] = p8(tk, s + 8u * (uint32_t) hb);
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const uint32_t at = s + 8u * (uint32_t) hb + (uint32_t) q;
                    if (8u * (uint32_t) hb + (uint32_t) q < r) {
#pragma unroll
                        for (int tk = 0; tk < (int) CP_TOK; ++tk) {
                            const float x = p[tk][q] * v[8 * hb + q];
                            acc[tk] = at < npast_t[tk] ? acc[tk] + x : acc[tk];
                        }
                    }
                }
            }
        }
    };
    load16(0, va);
    load16(16, vb);
    uint32_t s = 0;
    const uint32_t end = npast_max;
    const uint32_t bulk = min(end, npast_min);      // every token live before this
    for (; s + 32 <= bulk; s += 32) {
        step16(s, va);
        load16(s + 32, va);
        step16(s + 16, vb);
        load16(s + 48, vb);
    }
    // at most 15 + 3 positions remain, in va then vb
    if (s + 16 <= bulk) {
        step16(s, va);
        s += 16;
        load16(s + 16, va);
        tail(s, min(end - s, 16u), vb);
        if (end - s > 16) tail(s + 16, end - s - 16, va);
    } else {
        tail(s, min(end - s, 16u), va);
        if (end - s > 16) tail(s + 16, end - s - 16, vb);
    }
    if (64u * half_id + lane < hd) {
#pragma unroll
        for (int tk = 0; tk < (int) CP_TOK; ++tk) {
            const uint32_t t = tb + (uint32_t) tk;
            if (t < n_tok) A.out[(size_t) t * A.n_head * hd + (size_t) (kvh * grp + h) * hd + 64u * half_id + lane] = acc[tk];
        }
    }
}

// One workgroup of sixteen waves per CU (the host pads its LDS so that no
// second one fits). Units are numbered longest first (the last token blocks
// first) and dealt over the launch's SIMDs back and forth -- SIMD j of S
// takes units j, 2S - 1 - j, 2S + j, ... -- so that the SIMDs' sums of
// lengths agree to within a few percent. A wave reads which SIMD it runs on
// and takes that SIMD's units in order through a counter in LDS; once they
// are gone it helps with the other SIMDs' of its CU, so every unit is done
// whatever the placement of the waves.
extern "C" __global__ void __launch_bounds__(CP_THREADS)
sllm_k_chk_pv(dec_attn A, uint32_t n_tok) {
    __shared__ uint32_t s_next[4];
    const uint32_t lane = threadIdx.x & 63u;
    if (threadIdx.x < 4) s_next[threadIdx.x] = 0;
    __syncthreads();
    // HW_ID bits 5:4: the SIMD this wave runs on
    const uint32_t simd = __builtin_amdgcn_readfirstlane((__builtin_amdgcn_s_getreg(63492) >> 4) & 3u);
    const uint32_t n_simd = 4u * gridDim.x;
    const uint32_t grp = A.n_head / A.n_kv, halves = (A.hd + 63u) / 64u;
    const uint32_t per_tb = A.n_kv * grp * halves;                  // units per token block
    const uint32_t n_tb = (n_tok + CP_TOK - 1) / CP_TOK, n_units = per_tb * n_tb;
    for (uint32_t j = 0; j < 4u; ++j) {
        const uint32_t sm = (simd + j) & 3u, sig = 4u * blockIdx.x + sm;
        for (;;) {
            uint32_t r = 0;
            if (lane == 0) r = atomicAdd(&s_next[sm], 1u);
            r = __builtin_amdgcn_readfirstlane(r);
            const uint32_t k = r * n_simd + ((r & 1u) ? n_simd - 1u - sig : sig);
            if (k >= n_units) break;                                // uniform; later rounds are further out
            const uint32_t rem = k % per_tb, kh = rem / halves;
            chk_pv_unit(A, n_tok, kh / grp, (n_tb - 1u - k / per_tb) * CP_TOK, lane, kh % grp, rem % halves);
        }
    }
}

// Argmax keys of one logits row (the chunk's last token): workgroup w's key
// is the largest over rows w*256 + tid + k*gridDim.x*256, for
// sllm_k_dec_argmax to finish.
extern "C" __global__ void __launch_bounds__(256)
sllm_k_chk_keys(const float *__restrict__ logits, uint32_t n, uint64_t *__restrict__ partial) {
    __shared__ uint64_t red[4];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    uint64_t best = 0;
    for (uint32_t i = blockIdx.x * 256 + tid; i < n; i += gridDim.x * 256) {
        const uint64_t key = argmax_key(logits[i], i);
        best = key > best ? key : best;
    }
    best = wave_max_u64(best);
    if (lane == 0) red[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
        for (int i = 1; i < 4; ++i) best = red[i] > best ? red[i] : best;
        partial[blockIdx.x] = best;
    }
}

// Diagnostic (no counterpart in the reference): the softmax tail's expf
// (libm_expf.h, the C library's algorithm) on the device, for the float
// whose bit pattern is first + i * stride (mod 2^32), i < n -- so that a
// test can hold the device build against the host library's expf.
extern "C" __global__ void __launch_bounds__(256)
sllm_k_diag_expf(uint32_t first, uint32_t stride, uint32_t n, float *__restrict__ out) {
    __shared__ uint64_t tab[32];
    if (threadIdx.x < 32) tab[threadIdx.x] = c_expf_tab[threadIdx.x];
    __syncthreads();
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
        out[i] = sllm_libm_expf(__uint_as_float(first + i * stride), tab);
    }
}
