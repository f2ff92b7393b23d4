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
//   then       sllm_k_dec_lm_head          (residual, output_norm, F16 rows,
//                                           argmax, next token)
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
    uint64_t       key;         // running argmax key of the current step (0: none)
    uint32_t       ticket;      // lm_head workgroups done with the current step
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

// ggml_v_expf, one lane (src/ops.c:342-379): the lane's value does not depend
// on its neighbours, and the vector code's all-in-range shortcut returns what
// the blend gives such a lane.
__device__ __forceinline__ float ggml_v_expf(float x) {
    const float r = 0x1.8p23f;
    const float z = fmaf(x, 0x1.715476p+0f, r);
    const float n = z - r;
    const float b = fmaf(-n, 0x1.7f7d1cp-20f, fmaf(-n, 0x1.62e4p-1f, x));
    const uint32_t e = __float_as_uint(z) << 23;
    const float k = __uint_as_float(e + __float_as_uint(1.0f));
    const float u = b * b;
    const float j = fmaf(fmaf(fmaf(0x1.0e4020p-7f, b, 0x1.573e2ep-5f), u,
                              fmaf(0x1.555e66p-3f, b, 0x1.fffdb6p-2f)),
                         u, 0x1.ffffecp-1f * b);
    if (!(fabsf(n) > 126.0f)) return fmaf(j, k, k);
    const uint32_t g = n <= 0.0f ? 0x82000000u : 0u;
    const float s1 = __uint_as_float(g + 0x7f000000u);
    const float s2 = __uint_as_float(e - g);
    if (fabsf(n) > 192.0f) return s1 * s1;
    return fmaf(s2, j, s2) * s1;
}

__constant__ uint64_t c_expf_tab[32] = SLLM_EXPF_TAB_INIT;

// SiLU as src/ops.c:428-440 computes it in its eight-wide body
__device__ __forceinline__ float silu(float v) {
    return v / (1.0f + ggml_v_expf(0.0f - v));
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
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

// The workgroup's slab covers job d.job (gate) and the same rows of job
// d.job + 1 (up); it writes silu(gate) * up into the gate job's out_f.
constexpr uint32_t WG_PAIR = 2;

struct dec_shared {
    int8_t  q[SLAB_MAX_K];
    int32_t dots[SLAB_MAX_ROWS];
    double  red_d[SLAB_WAVES];
    double  lane_d[4];
    float   red_f[SLAB_WAVES];
    int     red_i[SLAB_WAVES];
};

template <int MODE>
__device__ __forceinline__ float stage_elem(const dec_stage &st, int32_t token, uint32_t j) {
    if (MODE == IN_EMBED) return embd_f32(((const uint16_t *) st.a)[(size_t) token * st.k + j]);
    float v = ((const float *) st.a)[j];
    if (MODE == IN_RESID) v = v + st.b[j];
    return v;
}

template <int LPR, int CPL, int XV, int QV, int MODE, bool PAIR>
__device__ __forceinline__ void dec_block(const dec_stage &st, const gemv_job *__restrict__ jobs,
                                          const wg_desc d, dec_shared &S) {
    constexpr uint32_t RPW = 64 / LPR;
    constexpr uint32_t G = SLAB_WAVES * RPW;
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane((uint32_t) tid >> 6);
    const gemv_job job0 = jobs[d.job];
    const gemv_job job1 = PAIR ? jobs[d.job + 1] : job0;
    const uint32_t k = job0.k, chunks = k >> 6, row_bytes = k >> 2;
    const uint32_t n_rows = job0.n_rows, last_row = n_rows - 1;
    const __amdgpu_buffer_rsrc_t rs0 = tensor_rsrc(job0), rs1 = tensor_rsrc(job1);
    const uint32_t n_groups = (n_rows + G - 1) / G;
    const uint32_t per = (n_groups + d.b - 1) / d.b;
    const uint32_t first = d.a * per;
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
    int ls = 0;
#pragma unroll
    for (int u = 0; u < XV; ++u) {
        const uint32_t i = 4u * (uint32_t) (tid + u * SLAB_THREADS);
        if (i < k) {
            const int a = quant_one(xn[u][0] * qs), b = quant_one(xn[u][1] * qs);
            const int c = quant_one(xn[u][2] * qs), e = quant_one(xn[u][3] * qs);
            ls += a + b + c + e;
            *reinterpret_cast<uint32_t *>(S.q + i) =
                (uint32_t) (a & 0xff) | ((uint32_t) (b & 0xff) << 8) |
                ((uint32_t) (c & 0xff) << 16) | ((uint32_t) (e & 0xff) << 24);
        }
    }
    ls = wave_sum(ls);
    if (lane == 0) S.red_i[wave] = ls;
    __syncthreads();
    int32_t asum = 0;
#pragma unroll
    for (int w = 0; w < SLAB_WAVES; ++w) asum += S.red_i[w];

    // (5) the row groups, double-buffered (as the slab kernel)
    int32_t *dots = S.dots + wave_row;
    uint32_t t = 0;
    for (uint32_t pair = 0; pair < TT / 2; ++pair) {
        slab_load<LPR, CPL>(group_rsrc(t + 1), row_bytes, group_row(t + 1), last_row, bufb);
        slab_dot<LPR, CPL>(chunks, group_row(t), n_rows, bufa, S.q, dots + t * G);
        ++t;
        slab_load<LPR, CPL>(group_rsrc(t + 1), row_bytes, group_row(t + 1), last_row, bufa);
        slab_dot<LPR, CPL>(chunks, group_row(t), n_rows, bufb, S.q, dots + t * G);
        ++t;
    }
    if (TT & 1u) slab_dot<LPR, CPL>(chunks, group_row(t), n_rows, bufa, S.q, dots + t * G);
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
    if (d.flags & WG_PUBLISH) {
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

template <int LPR, int CPL, int XV, int QV>
__device__ __forceinline__ void dec_variant(const dec_stage &st, const gemv_job *jobs, const wg_desc d,
                                            dec_shared &S) {
    const bool pair = (d.flags & WG_PAIR) != 0;
    switch (st.mode) {
    case IN_EMBED:
        if (pair) dec_block<LPR, CPL, XV, QV, IN_EMBED, true>(st, jobs, d, S);
        else dec_block<LPR, CPL, XV, QV, IN_EMBED, false>(st, jobs, d, S);
        break;
    case IN_RESID:
        if (pair) dec_block<LPR, CPL, XV, QV, IN_RESID, true>(st, jobs, d, S);
        else dec_block<LPR, CPL, XV, QV, IN_RESID, false>(st, jobs, d, S);
        break;
    default:
        if (pair) dec_block<LPR, CPL, XV, QV, IN_PLAIN, true>(st, jobs, d, S);
        else dec_block<LPR, CPL, XV, QV, IN_PLAIN, false>(st, jobs, d, S);
        break;
    }
}

// ---------------------------------------------------------------------------
// attention (src/forward.c:668-726): RoPE (NeoX pairs, cos/sin from a table
// the host builds with the reference's libm calls), KV store, scores.
// ---------------------------------------------------------------------------

struct dec_attn {
    const float    *q, *k, *v;          // projections: q [n_head*hd], k / v [n_kv*hd]
    float          *k_cache, *v_cache;  // this layer's caches [n_kv][n_ctx][hd]
    const float    *rope;               // [n_ctx][half] (cos, sin)
    float          *scores;             // [n_head][n_ctx]
    float          *out;                // [n_head*hd]
    const dec_step *step;
    float           attn_scale;
    uint32_t        n_head, n_kv, hd, half, n_ctx;
    uint32_t        pad;
};
static_assert(sizeof(dec_attn) == 104, "dec_attn must match decode.c");

constexpr int ATT_THREADS = 256;
constexpr uint32_t ATT_POS = 64;        // positions per scores workgroup
constexpr uint32_t ATT_MAX_HD = 128;
constexpr uint32_t ATT_MAX_GRP = 8;     // query heads per KV head
constexpr uint32_t PV_SLICE = 16;       // head dimensions per p.V workgroup
constexpr uint32_t PV_CHUNK = 256;      // positions of V staged per pass
constexpr uint32_t PV_MAX_P = 16384;    // query heads per KV head x positions

// element d of a head vector after NeoX RoPE (src/ops.c:467-549): pairs
// (e, e + half) rotate by angle e; dimensions from 2*half on pass through
__device__ __forceinline__ float rope_at(const float *x, uint32_t d, uint32_t half, const float *cs) {
    if (d < half) return x[d] * cs[2 * d] - x[d + half] * cs[2 * d + 1];
    if (d < 2 * half) {
        const uint32_t e = d - half;
        return x[e] * cs[2 * e + 1] + x[d] * cs[2 * e];
    }
    return x[d];
}

} // namespace

// ---------------------------------------------------------------------------
// entry points (argument lists mirrored in decode.c)
// ---------------------------------------------------------------------------

// One decode GEMV stage. Variant 0 (K <= 2560): 8 lanes per row; variant 1
// (K <= 7168): 16 lanes per row.
extern "C" __global__ void __launch_bounds__(SLAB_THREADS)
sllm_k_dec_gemv(const dec_stage *__restrict__ stage, const gemv_job *__restrict__ jobs,
                const wg_desc *__restrict__ descs, uint32_t n_wg) {
    __shared__ dec_shared S;
    const wg_desc d = descs[xcd_slot(n_wg)];
    if (d.b == 0) return;
    const dec_stage st = *stage;
    if (jobs[d.job].variant == 0) dec_variant<8, 5, 3, 1>(st, jobs, d, S);
    else dec_variant<16, 7, 7, 2>(st, jobs, d, S);
}

// Scores: workgroup (KV head, 64 positions). Every workgroup ropes the query
// heads of its KV head; the one holding position pos ropes the new key and
// stores it, with the new value, into the caches (src/forward.c:668-690).
// Thread (h, r) then takes q_h . k_r over d in order, times 1/sqrt(hd)
// (src/forward.c:698-705).
extern "C" __global__ void __launch_bounds__(ATT_THREADS)
sllm_k_dec_scores(dec_attn A) {
    __shared__ float qr[ATT_MAX_GRP][ATT_MAX_HD];
    __shared__ float kt[ATT_POS][ATT_MAX_HD + 1];
    const uint32_t kvh = blockIdx.x, s0 = blockIdx.y * ATT_POS, tid = threadIdx.x;
    const uint32_t pos = (uint32_t) A.step->pos, npast = pos + 1;
    if (s0 >= npast) return;
    const uint32_t grp = A.n_head / A.n_kv, hd = A.hd, half = A.half;
    const float *cs = A.rope + (size_t) pos * half * 2;
    for (uint32_t idx = tid; idx < grp * hd; idx += ATT_THREADS) {
        const uint32_t hh = idx / hd, d = idx % hd;
        qr[hh][d] = rope_at(A.q + (size_t) (kvh * grp + hh) * hd, d, half, cs);
    }
    const uint32_t n_here = min(ATT_POS, npast - s0);
    float *kc = A.k_cache + (size_t) kvh * A.n_ctx * hd;
    float *vc = A.v_cache + (size_t) kvh * A.n_ctx * hd;
    for (uint32_t idx = tid; idx < n_here * hd; idx += ATT_THREADS) {
        const uint32_t r = idx / hd, d = idx % hd, s = s0 + r;
        float val;
        if (s < pos) {
            val = kc[(size_t) s * hd + d];
        } else {
            val = rope_at(A.k + (size_t) kvh * hd, d, half, cs);
            kc[(size_t) pos * hd + d] = val;
            vc[(size_t) pos * hd + d] = A.v[(size_t) kvh * hd + d];
        }
        kt[r][d] = val;
    }
    __syncthreads();
    const uint32_t r = tid % ATT_POS;
    if (r < n_here) {
        for (uint32_t hh = tid / ATT_POS; hh < grp; hh += ATT_THREADS / ATT_POS) {
            float acc = 0.0f;
            for (uint32_t d = 0; d < hd; ++d) acc = acc + qr[hh][d] * kt[r][d];
            A.scores[(size_t) (kvh * grp + hh) * A.n_ctx + s0 + r] = acc * A.attn_scale;
        }
    }
}

// Softmax and p . V: workgroup (KV head, 16 head dimensions). Wave w takes
// the softmax of query heads w, w + 4, ... of the KV head (src/ops.c:386-422:
// max; ggml_v_expf over whole groups of eight, the C library's expf over the
// rest; the double sum, each eight-group added as ((t0 + t1) + t2) + t3 of
// t_j = e_j + e_{j+4}; 1/sum narrowed to f32; p = e * inv). Then thread
// (h, dd) accumulates p_s * v_s over s = 0..pos in order
// (src/forward.c:706-726), V staged through LDS.
extern "C" __global__ void __launch_bounds__(ATT_THREADS)
sllm_k_dec_pv(dec_attn A) {
    __shared__ float P[PV_MAX_P];
    __shared__ float vs[2][PV_CHUNK][PV_SLICE];
    __shared__ float inv_h[ATT_MAX_GRP];
    const uint32_t kvh = blockIdx.x, d0 = blockIdx.y * PV_SLICE, tid = threadIdx.x;
    const uint32_t lane = tid & 63, wave = tid >> 6;
    const uint32_t npast = (uint32_t) A.step->pos + 1;
    const uint32_t grp = A.n_head / A.n_kv, hd = A.hd;
    const uint32_t nb = npast / 8, nt = nb * 8;

    // exponentials
    for (uint32_t hh = wave; hh < grp; hh += ATT_THREADS / 64) {
        const float *sc = A.scores + (size_t) (kvh * grp + hh) * A.n_ctx;
        float *p = P + hh * npast;
        float m = -INFINITY;
        for (uint32_t s = lane; s < npast; s += 64) m = fmaxf(m, sc[s]);
        m = wave_max(m);
        for (uint32_t s = lane; s < npast; s += 64) {
            const float x = sc[s] - m;
            p[s] = s < nt ? ggml_v_expf(x) : sllm_libm_expf(x, c_expf_tab);
        }
    }
    __syncthreads();

    // sums: any order, checked; the reference's order when the check fails
    auto block_sum = [](const float *e) {
        const double t0 = (double) e[0] + (double) e[4], t1 = (double) e[1] + (double) e[5];
        const double t2 = (double) e[2] + (double) e[6], t3 = (double) e[3] + (double) e[7];
        return ((t0 + t1) + t2) + t3;
    };
    for (uint32_t hh = wave; hh < grp; hh += ATT_THREADS / 64) {
        const float *p = P + hh * npast;
        double part = 0.0;
        for (uint32_t b = lane; b < nb; b += 64) part += block_sum(p + 8 * b);
        if (lane == 0) {
            for (uint32_t s = nt; s < npast; ++s) part += (double) p[s];
        }
        const double sum = wave_sum_d(part);
        const double bound = sum * ((double) (nb + (npast - nt) + 8) * 0x1p-52);
        float inv = (float) (1.0 / (sum - bound));
        if (inv != (float) (1.0 / (sum + bound))) {   // uniform over the wave
            if (lane == 0) {
                double seq = 0.0;
                for (uint32_t b = 0; b < nb; ++b) seq += block_sum(p + 8 * b);
                for (uint32_t s = nt; s < npast; ++s) seq += (double) p[s];
                inv = (float) (1.0 / seq);
            }
            inv = __shfl(inv, 0, 64);
        }
        if (lane == 0) inv_h[hh] = inv;
    }
    __syncthreads();
    for (uint32_t i = tid; i < grp * npast; i += ATT_THREADS) P[i] = P[i] * inv_h[i / npast];

    // p . V: V[s][d0 .. d0+16) staged PV_CHUNK positions at a time
    const float *vc = A.v_cache + (size_t) kvh * A.n_ctx * hd + d0;
    const uint32_t chains = grp * PV_SLICE;
    const uint32_t hh = tid / PV_SLICE, dd = tid % PV_SLICE;
    const uint32_t n_chunks = (npast + PV_CHUNK - 1) / PV_CHUNK;
    f32x4 stage[4];
    auto load_chunk = [&](uint32_t c) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t idx = tid + (uint32_t) u * ATT_THREADS, r = idx / 4, c4 = idx % 4;
            const uint32_t s = min(c * PV_CHUNK + r, npast - 1);
            stage[u] = *G_CAST(const f32x4, vc + (size_t) s * hd + 4 * c4);
        }
    };
    auto store_chunk = [&](uint32_t buf) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t idx = tid + (uint32_t) u * ATT_THREADS, r = idx / 4, c4 = idx % 4;
            *reinterpret_cast<f32x4 *>(&vs[buf][r][4 * c4]) = stage[u];
        }
    };
    load_chunk(0);
    __syncthreads();                 // P normalised everywhere
    store_chunk(0);
    __syncthreads();
    float acc = 0.0f;
    for (uint32_t c = 0; c < n_chunks; ++c) {
        if (c + 1 < n_chunks) load_chunk(c + 1);
        if (tid < chains) {
            const float *p = P + hh * npast + c * PV_CHUNK;
            const uint32_t n = min(PV_CHUNK, npast - c * PV_CHUNK);
            for (uint32_t r = 0; r < n; ++r) acc = acc + p[r] * vs[c & 1][r][dd];
        }
        if (c + 1 < n_chunks) store_chunk((c + 1) & 1);
        __syncthreads();
    }
    if (tid < chains) A.out[(size_t) (kvh * grp + hh) * hd + d0 + dd] = acc;
}

// ---------------------------------------------------------------------------
// output: x = a + b, RMSNorm with output_norm, the F16 rows
// (src/forward.c:800-827), argmax (src/forward.c:876-883) and the next token
// ---------------------------------------------------------------------------

struct dec_lm {
    const float    *a, *b;       // the final residual is a + b
    const float    *norm_w;
    const uint16_t *embd;        // [n_vocab][n_embd] f16, the tied output projection
    float          *logits;
    dec_step       *step;
    float           eps;
    uint32_t        n_embd, n_vocab, pad;
};
static_assert(sizeof(dec_lm) == 64, "dec_lm must match decode.c");

constexpr int LM_THREADS = 256;
constexpr uint32_t LM_ROWS = 64;        // four lanes per row
constexpr uint32_t LM_MAX_E = 8192;
constexpr int LM_UNROLL = 8;

// Row . xn as src/ops.c:106-154 orders it: lane j of a row's four holds
// acc[j][0..7], element 32i + 8j + l going into acc[j][l] by FMA; then
// acc0 += acc2, acc1 += acc3, acc0 += acc1; t_l = acc0[l] + acc0[l+4];
// (t0 + t1) + (t2 + t3). n_embd % 32 == 0, so there is no scalar tail.
extern "C" __global__ void __launch_bounds__(LM_THREADS)
sllm_k_dec_lm_head(dec_lm L) {
    __shared__ __attribute__((aligned(16))) float xn[LM_MAX_E];
    __shared__ double red_d[LM_THREADS / 64], lane_d[4];
    __shared__ uint64_t red_k[LM_THREADS / 64];
    const uint32_t e = L.n_embd, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    double part = 0.0;
    for (uint32_t i = tid; i < e; i += LM_THREADS) {
        const float v = L.a[i] + L.b[i];
        xn[i] = v;
        part += (double) (v * v);
    }
    const float mean = rms_mean(part, e, red_d, lane_d, [&](uint32_t j) { return L.a[j] + L.b[j]; });
    const float scale = 1.0f / sqrtf(mean + L.eps);
    for (uint32_t i = tid; i < e; i += LM_THREADS) xn[i] = (scale * xn[i]) * L.norm_w[i];
    __syncthreads();

    const uint32_t row = blockIdx.x * LM_ROWS + wave * 16 + lane / 4, j = lane % 4;
    const bool valid = row < L.n_vocab;
    const GLOBAL u32x4 *w = G_CAST(const u32x4, L.embd + (size_t) (valid ? row : L.n_vocab - 1) * e) + j;
    const uint32_t steps = e / 32;
    float acc[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
    for (uint32_t i0 = 0; i0 < steps; i0 += LM_UNROLL) {
        u32x4 h[LM_UNROLL];
#pragma unroll
        for (int u = 0; u < LM_UNROLL; ++u) h[u] = __builtin_nontemporal_load(w + 4 * min(i0 + u, steps - 1));
#pragma unroll
        for (int u = 0; u < LM_UNROLL; ++u) {
            if (i0 + u < steps) {
                const f32x8 hf = __builtin_convertvector(__builtin_bit_cast(f16x8, h[u]), f32x8);
                const float *x = xn + 32 * (i0 + u) + 8 * j;
#pragma unroll
                for (int l = 0; l < 8; ++l) acc[l] = fmaf(hf[l], x[l], acc[l]);
            }
        }
    }
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = acc[l] + __shfl_xor(acc[l], 2, 64);   // acc0 += acc2, acc1 += acc3
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = acc[l] + __shfl_xor(acc[l], 1, 64);   // acc0 += acc1
    const float t0 = acc[0] + acc[4], t1 = acc[1] + acc[5], t2 = acc[2] + acc[6], t3 = acc[3] + acc[7];
    const float s = (t0 + t1) + (t2 + t3);

    uint64_t key = 0;
    if (valid && j == 0) {
        G_CAST(float, L.logits)[row] = s;
        if (!__builtin_isnan(s)) {
            const uint32_t u = __float_as_uint(s == 0.0f ? 0.0f : s);       // -0 ties with +0
            const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
            key = ((uint64_t) ord << 32) | (uint64_t) (0xffffffffu - row);  // the first index wins ties
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint64_t other = __shfl_xor(key, o, 64);
        key = other > key ? other : key;
    }
    if (lane == 0) red_k[wave] = key;
    __syncthreads();
    if (tid == 0) {
        uint64_t k = red_k[0];
        for (int i = 1; i < LM_THREADS / 64; ++i) k = red_k[i] > k ? red_k[i] : k;
        dec_step *st = L.step;
        atomicMax((unsigned long long *) &st->key, (unsigned long long) k);
        __threadfence();
        const uint32_t done = atomicAdd(&st->ticket, 1u);
        if (done == gridDim.x - 1) {
            // the last workgroup: every row's logit and key are in
            __threadfence();
            const uint64_t best = __hip_atomic_load(&st->key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            int32_t next = best == 0 ? 0 : (int32_t) (0xffffffffu - (uint32_t) best);
            const float l0 = __hip_atomic_load(L.logits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (__builtin_isnan(l0)) next = 0;      // a NaN first logit is never beaten
            st->next = next;
            st->key = 0;
            st->ticket = 0;
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
    }
}
