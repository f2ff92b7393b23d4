// i2s_kernels.hip -- gfx950 device code for the I2_S ternary path.
//
// Built with `hipcc --genco --offload-arch=gfx950` into a code object that the
// C11 shim (gfx950_shim.c) loads with hipModuleLoadData and launches with
// hipModuleLaunchKernel. Only extern "C" __global__ entry points are visible to
// the shim; their argument lists are mirrored there.
//
// Packed I2_S tensor, exactly as stored in the GGUF (src/quant.c:72-106,
// FORMAT.md:119-157): an N x K matrix is N rows of K/4 bytes, row r at byte
// r*K/4, followed by a 32-byte tail whose first 4 bytes are the f32 per-tensor
// scale (offset N*K/4). Within a row, 128-element block b is 32 bytes at 32*b;
// byte l of the block holds elements 128*b + 32*f + l for fields f = 0..3 at
// bit shift 6 - 2*f (field 0 in the top two bits). Codes {0,1,2} stand for
// ternary {-1,0,+1}. The kernels read this layout directly: nothing is
// repacked on upload.
//
// Arithmetic contract (src/i2s_gemm.c:45-290, Makefile:16-41): int8
// activations and int32 dot products are exact; float work is IEEE single
// with correctly rounded division, no contraction and no denormal flushing,
// so every float result is the same bits the C reference produces.

#include "i2s_device.h"


namespace {

// LPR lanes per row, CPL chunks per lane (LPR * CPL * 64 >= K), XV f32x4 and
// QV 16-byte activation loads per thread (covering K). QUANT: the job carries
// f32 x (quantised here) rather than a quantised row; it is a template
// argument so that each instantiation is one straight path and the compiler
// never has to assume the other input's loads might still be in flight.
//
// A job's rows are cut into groups of G = 4 * 64/LPR rows, one per pass of
// the workgroup's four waves; slab a of b takes the a-th run of consecutive
// groups. (Dealing the groups round-robin instead, so that a job's slabs
// sweep it side by side, measured no faster.)
template <int LPR, int CPL, int XV, int QV, bool QUANT>
__device__ __forceinline__ void slab_block(const gemv_job &job, uint32_t slab, uint32_t n_slabs,
                                           uint32_t flags, slab_shared &S) {
    constexpr uint32_t RPW = 64 / LPR;
    constexpr uint32_t G = SLAB_WAVES * RPW;
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane((uint32_t) tid >> 6);
    const uint32_t k = job.k, row_bytes = k >> 2;
    const uint32_t n_rows = job.n_rows, last_row = n_rows - 1;
    const __amdgpu_buffer_rsrc_t rsrc = tensor_rsrc(job);
    // this slab's groups: first .. first + T - 1
    const uint32_t n_groups = (n_rows + G - 1) / G;
    const uint32_t per = (n_groups + n_slabs - 1) / n_slabs;
    const uint32_t first = slab * per;
    const uint32_t T = first < n_groups ? min(per, n_groups - first) : 0u;
    if (T == 0) return;                        // uniform: no group here
    // the wave's first row in its t-th group; past the end, the last group again
    const uint32_t wave_row = wave * RPW;
    auto group_row = [&](uint32_t t) { return (first + min(t, T - 1)) * G + wave_row; };

    // (1) the activation first -- f32 x to quantise here, or the int8 row --
    // so that waiting for it leaves the weight loads behind it in flight
    f32x4 xv[XV];
    u32x4 qv[QV];
    float scale = 0.0f;
    int32_t asum = 0, a2 = 0;       // a2: twice the sum of the row's field-0 elements (slab_dot_x)
    if (QUANT) {
#pragma unroll
        for (int u = 0; u < XV; ++u) {
            const uint32_t i = 4u * (uint32_t) (tid + u * SLAB_THREADS);
            xv[u] = *G_CAST(const f32x4, job.x + min(i, k - 4));
        }
    } else {
#pragma unroll
        for (int u = 0; u < QV; ++u) {
            const uint32_t i = 16u * (uint32_t) (tid + u * SLAB_THREADS);
            qv[u] = *G_CAST(const u32x4, job.q + min(i, k - 16));
        }
        // act is optional without an epilogue; read a valid address either way
        const GLOBAL int32_t *ap = G_CAST(const int32_t, job.act != nullptr ? (const void *) job.act
                                                                          : (const void *) job.w);
        const float sc = __int_as_float(ap[0]);
        const int32_t sm = ap[1];
        scale = job.act != nullptr ? sc : 0.0f;
        asum = job.act != nullptr ? sm : 0;
    }
    // w_scale for the epilogue; without one, read row 0 instead of a tail
    // the caller need not have given (no branch around the load)
    const uint8_t *ws_at = job.out_f != nullptr ? job.w + (size_t) job.n_rows * row_bytes : job.w;
    const float ws = G_CAST(const float, ws_at)[vzero()];   // a vector load
    // keep the scheduler from moving activation loads behind the weight loads
    __builtin_amdgcn_sched_barrier(0);

    // (2) the wave's first row group
    u32x4 bufa[CPL], bufb[CPL];
    slab_load<LPR, CPL>(rsrc, row_bytes, group_row(0), last_row, bufa);

    // (3) the activation into LDS
    if (QUANT) {
        float m = 0.0f;        // fmaxf drops NaN exactly as the reference's `a > amax` does
#pragma unroll
        for (int u = 0; u < XV; ++u) {
            const uint32_t i = 4u * (uint32_t) (tid + u * SLAB_THREADS);
            const f32x4 v = xv[u];
            const float a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
            m = fmaxf(m, i < k ? a : 0.0f);
        }
        m = wave_max(m);
        if (lane == 0) S.red_f[wave] = m;
        __syncthreads();
        m = S.red_f[0];
#pragma unroll
        for (int w = 1; w < SLAB_WAVES; ++w) m = fmaxf(m, S.red_f[w]);
        const float s = m > 0.0f ? 127.0f / m : 0.0f;
        int ls = 0, la = 0;
#pragma unroll
        for (int u = 0; u < XV; ++u) {
            const uint32_t i = 4u * (uint32_t) (tid + u * SLAB_THREADS);
            if (i < k) {
                const f32x4 v = xv[u];
                const int a = quant_one(v[0] * s), b = quant_one(v[1] * s);
                const int c = quant_one(v[2] * s), d = quant_one(v[3] * s);
                ls += a + b + c + d;
                la += ((i >> 5) & 3u) == 0 ? a + b + c + d : 0;     // field 0 of its block
                *reinterpret_cast<uint32_t *>(S.q + i) =
                    (uint32_t) (a & 0xff) | ((uint32_t) (b & 0xff) << 8) |
                    ((uint32_t) (c & 0xff) << 16) | ((uint32_t) (d & 0xff) << 24);
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
        int t = 0, ta = 0;
#pragma unroll
        for (int w = 0; w < SLAB_WAVES; ++w) {
            t += S.red_i[w];
            ta += S.red_a[w];
        }
        scale = s;
        asum = t;
        a2 = 2 * ta;
    } else {
        int la = 0;
#pragma unroll
        for (int u = 0; u < QV; ++u) {
            const uint32_t i = 16u * (uint32_t) (tid + u * SLAB_THREADS);
            const u32x4 zero = { 0, 0, 0, 0 };
            if (i < SLAB_MAX_K) *reinterpret_cast<u32x4 *>(S.q + i) = i < k ? qv[u] : zero;
            if (i < k && ((i >> 5) & 3u) == 0) {
#pragma unroll
                for (int d = 0; d < 4; ++d) la = __builtin_amdgcn_sdot4((int) qv[u][d], 0x01010101, la, false);
            }
        }
        la = wave_sum(la);
        if (lane == 0) S.red_a[wave] = la;
        __syncthreads();
        int ta = 0;
#pragma unroll
        for (int w = 0; w < SLAB_WAVES; ++w) ta += S.red_a[w];
        a2 = 2 * ta;
    }

    // (4) the groups, double-buffered: pairs of groups with the next group
    // always loaded before the current one is reduced, then a trailing odd
    // group. The load past the last group goes to the dead offset (no memory
    // read). The loop has one exit and no load behind a branch, so every wait
    // names exactly the buffer it needs. Dots of group t go to S.dots[t*G ..].
    int32_t *dots = S.dots + wave_row;
    uint32_t t = 0;
    for (uint32_t pair = 0; pair < T / 2; ++pair) {
        slab_load<LPR, CPL>(rsrc, row_bytes, group_row(t + 1), last_row, bufb, t + 1 < T);
        slab_dot_x<LPR, CPL>(group_row(t), n_rows, bufa, S.q, a2, dots + t * G);
        ++t;
        slab_load<LPR, CPL>(rsrc, row_bytes, group_row(t + 1), last_row, bufa, t + 1 < T);
        slab_dot_x<LPR, CPL>(group_row(t), n_rows, bufb, S.q, a2, dots + t * G);
        ++t;
    }
    if (T & 1u) slab_dot_x<LPR, CPL>(group_row(t), n_rows, bufa, S.q, a2, dots + t * G);
    __syncthreads();

    // (5) raw dots and the epilogue (src/i2s_gemm.c:271-290): post once per
    // column, then (float)(dot - sum) * post per row
    const float post = job.out_f != nullptr ? ws / scale : 0.0f;
    for (uint32_t i = (uint32_t) tid; i < T * G; i += SLAB_THREADS) {
        const uint32_t row = first * G + i;
        if (row < n_rows) {
            const int32_t d = S.dots[i];
            if (job.out_i != nullptr) G_CAST(int32_t, job.out_i)[row] = d;
            if (job.out_f != nullptr) G_CAST(float, job.out_f)[row] = (float) (d - asum) * post;
        }
    }

    // (6) one workgroup of the job publishes the row it quantised
    if ((flags & WG_PUBLISH) && QUANT) {
        if (job.q != nullptr) {
#pragma unroll
            for (int u = 0; u < QV; ++u) {
                const uint32_t i = 16u * (uint32_t) (tid + u * SLAB_THREADS);
                if (i < k) *G_CAST(u32x4, job.q + i) = *reinterpret_cast<const u32x4 *>(S.q + i);
            }
        }
        if (job.act != nullptr && tid == 0) {
            G_CAST(float, job.act)[0] = scale;
            G_CAST(int32_t, job.act)[1] = asum;
        }
    }
}

// ---------------------------------------------------------------------------
// streaming GEMV (any K up to the LDS limit): waves loop over row groups with
// UNROLL loads in flight per lane, reading a quantised activation staged in
// LDS (x must be null: the plan quantises such jobs first).
// ---------------------------------------------------------------------------

constexpr int UNROLL = 8;

template <int LPR>
__device__ __forceinline__ void stream_rows(const gemv_job &job, uint32_t row_begin,
                                            uint32_t row_end, const int8_t *q_lds,
                                            int32_t asum, float post) {
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int wave = (int) __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), waves = blockDim.x >> 6;
    const int sub = lane % LPR;
    const uint32_t k = job.k, chunks = k >> 6, row_bytes = k >> 2;

    for (uint32_t r0 = row_begin + (uint32_t) wave * RPW; r0 < row_end; r0 += (uint32_t) waves * RPW) {
        const uint32_t row = r0 + (uint32_t) (lane / LPR);
        const bool valid = row < row_end;
        const GLOBAL u32x4 *wr = G_CAST(const u32x4, job.w + (size_t) (valid ? row : row_begin) * row_bytes);
        dot4acc acc = { 0, 0, 0, 0 };
        if (valid) {
            for (uint32_t c0 = (uint32_t) sub; c0 < chunks; c0 += UNROLL * LPR) {
                u32x4 wv[UNROLL];
#pragma unroll
                for (int u = 0; u < UNROLL; ++u) {
                    const uint32_t c = c0 + (uint32_t) (u * LPR);
                    if (c < chunks) wv[u] = __builtin_nontemporal_load(wr + c);
                }
#pragma unroll
                for (int u = 0; u < UNROLL; ++u) {
                    const uint32_t c = c0 + (uint32_t) (u * LPR);
                    if (c < chunks) chunk_dot(wv[u], q_lds + (c >> 1) * 128u + (c & 1u) * 16u, acc);
                }
            }
        }
        const int dot = group_sum<LPR>(finish(acc));
        if (valid && sub == 0) {
            if (job.out_i != nullptr) G_CAST(int32_t, job.out_i)[row] = dot;
            if (job.out_f != nullptr) G_CAST(float, job.out_f)[row] = (float) (dot - asum) * post;
        }
    }
}

template <int LPR>
__device__ __forceinline__ void stream_block(const gemv_job &job, uint32_t row_begin, uint32_t row_end) {
    extern __shared__ __attribute__((aligned(16))) int8_t q_lds[];
    const uint32_t k = job.k;
    const uint32_t step = 16u * blockDim.x;
    // stage the activation: four loads in flight per thread between waits
    for (uint32_t i0 = 16u * threadIdx.x; i0 < k; i0 += 4u * step) {
        u32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t i = i0 + (uint32_t) u * step;
            if (i < k) v[u] = *G_CAST(const u32x4, job.q + i);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t i = i0 + (uint32_t) u * step;
            if (i < k) *reinterpret_cast<u32x4 *>(q_lds + i) = v[u];
        }
    }
    float post = 0.0f;
    int32_t asum = 0;
    if (job.out_f != nullptr) {
        post = tensor_scale(job) / G_CAST(const float, job.act)[0];
        asum = G_CAST(const int32_t, job.act)[1];
    }
    __syncthreads();
    stream_rows<LPR>(job, row_begin, row_end, q_lds, asum, post);
}

// A streaming workgroup's job and rows: from the descriptor table, or -- for
// a single-job launch (descs null) -- rows [blockIdx.x * single_rows, +single_rows)
// of `single`.
__device__ __forceinline__ bool stream_share(const gemv_job *__restrict__ jobs,
                                             const wg_desc *__restrict__ descs, uint32_t n_wg,
                                             const gemv_job &single, uint32_t single_rows,
                                             gemv_job &job, uint32_t &row_begin, uint32_t &row_end) {
    if (descs != nullptr) {
        const wg_desc d = descs[xcd_slot(n_wg)];
        if (d.a >= d.b) return false;
        job = jobs[d.job];
        row_begin = d.a;
        row_end = d.b;
        return true;
    }
    job = single;
    row_begin = blockIdx.x * single_rows;
    row_end = min(single.n_rows, row_begin + single_rows);
    return row_begin < row_end;
}


// ---------------------------------------------------------------------------
// batched ternary GEMM on int8 MFMA (several tokens against one tensor: the
// projections of a chunk, src/forward.c:589-793 with n > 1)
// ---------------------------------------------------------------------------
//
// C[t][n] = sum_k q[t][k] * code[n][k] with v_mfma_i32_16x16x64_i8: A = 16
// tokens x 64 k, B = 64 k x 16 rows. Lane l holds A[l % 16][16 (l/16) ..
// + 15] and B[16 (l/16) .. + 15][l % 16] and receives C[4 (l/16) + r][l % 16]
// (r = 0..3). The 64 k of one instruction are chosen to fit the I2_S layout:
// half h of 128-element block b, all four fields -- lane group g takes field
// g, elements 128 b + 32 g + 16 h + (0..15) -- so a lane's B operand is
// field g of the same 16 packed bytes the other three lane groups read,
// isolated in place (values 0..2, one per byte), and its A operand is 16
// consecutive int8 of the token's row. Integer sums do not depend on the
// order of k, so the dots are exactly the reference's.
//
// A workgroup is four waves side by side along the rows; each wave owns TM
// token tiles x TN row tiles (16 x 16 each), with the next k step's loads in
// flight while the current step's MFMAs run. No LDS.

typedef int32_t i32x4v __attribute__((ext_vector_type(4)));

// Up to three tensors of the same K against the same quantised rows (Q, K
// and V; gate and up): the grid's row tiles are job 0's, then job 1's, then
// job 2's.
struct gemm_args {
    const int8_t    *q;          // [m][k] int8
    const act_t     *act;        // [m]
    const uint8_t   *w[3];       // packed tensors with their tails
    float           *out[3];     // [m][n_rows] epilogue, or null
    int32_t         *out_i[3];   // [m][n_rows] raw dots, or null
    uint32_t         n_rows[3];
    uint32_t         tiles[3];   // row tiles (workgroups along x) of each job
    uint32_t         k, m, n_jobs, pad;
};

// the job of this workgroup's row tile, and the tile's index within it
struct gemm_view {
    const uint8_t *w;
    float         *out;
    int32_t       *out_i;
    uint32_t       n_rows, tile;
    const int8_t  *q;
    const act_t   *act;
    uint32_t       job;
    const uint8_t *w2;          // a gate + up tile: the up tensor (w is gate's)
    const float   *res;         // a residual tile: [m][n_rows] added to the output
};

// A chunk's Q + K + V launch (jobs 0, 1, 2 of gemm_args) that also does the
// attention's cache store (src/forward.c:668-690): queries and keys roped
// at their positions (NeoX, src/ops.c:467-549), the queries in place in
// out[0], the keys into the key cache, the values into the value cache.
// Token t of the launch sits at position pos0 + t. The host uses it only
// where a row tile holds whole heads (BN % hd == 0) and half % 4 == 0.
struct gemm_rope {
    const float *rope;          // [n_ctx][half] (cos, sin)
    float       *k_cache;       // [n_kv][hd / 8][n_ctx][8]
    float       *v_cache;       // [n_kv][hd / 8][n_ctx][8]
    uint32_t     n_ctx, hd, half, pos0;
};
static_assert(sizeof(gemm_rope) == 40, "gemm_rope must match gfx950_shim.c");

// One tensor of a GEMM plan (gemm_table): its own token rows, K and
// outputs; tile0 is its first row tile in the plan (mirrored in
// gfx950_shim.c).
struct gemm_tjob {
    const uint8_t *w;
    const int8_t  *q;            // [m][k] int8
    const act_t   *act;          // [m], or null without an epilogue
    float         *out;          // [m][n_rows] epilogue, or null
    int32_t       *out_i;        // [m][n_rows] raw dots, or null
    uint32_t       n_rows, k, tile0, pad;
};

struct gemm_table {
    const gemm_tjob *jobs;
    const uint32_t  *tile_job;   // row tile -> job
    uint32_t         m, pad;
};

__device__ __forceinline__ gemm_view gemm_pick(const gemm_args &G, uint32_t b = blockIdx.x) {
    const uint32_t t0 = G.tiles[0], t01 = t0 + G.tiles[1];
    const uint32_t j = b < t0 ? 0u : (b < t01 ? 1u : 2u);       // uniform; selects, no indexing
    return { j == 0 ? G.w[0] : (j == 1 ? G.w[1] : G.w[2]),
             j == 0 ? G.out[0] : (j == 1 ? G.out[1] : G.out[2]),
             j == 0 ? G.out_i[0] : (j == 1 ? G.out_i[1] : G.out_i[2]),
             j == 0 ? G.n_rows[0] : (j == 1 ? G.n_rows[1] : G.n_rows[2]),
             b - (j == 0 ? 0u : (j == 1 ? t0 : t01)), G.q, G.act, j };
}

template <int TM, int TN>
__device__ __forceinline__ void gemm_load(const gemm_args &G, const gemm_view &V, uint32_t t0, uint32_t n0,
                                          uint32_t step, i32x4v (&a)[TM], u32x4 (&b)[TN]) {
    const int lane = threadIdx.x & 63, g = lane >> 4, li = lane & 15;
    const uint32_t blk = step >> 1, h = step & 1u;
    const uint32_t kq = 128u * blk + 32u * (uint32_t) g + 16u * h;        // A: k offset of this lane group
    const uint32_t kw = 32u * blk + 16u * h;                              // B: byte offset in the row
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
        const uint32_t t = min(t0 + 16u * (uint32_t) tm + (uint32_t) li, G.m - 1);
        a[tm] = *G_CAST(const i32x4v, G.q + (size_t) t * G.k + kq);
    }
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
        const uint32_t n = min(n0 + 16u * (uint32_t) tn + (uint32_t) li, V.n_rows - 1);
        b[tn] = __builtin_nontemporal_load(G_CAST(const u32x4, V.w + (size_t) n * (G.k >> 2) + kw));
    }
}

template <int TM, int TN>
__device__ __forceinline__ void gemm_mma(const i32x4v (&a)[TM], const u32x4 (&b)[TN], i32x4v (&c)[TM][TN]) {
    const int g = (threadIdx.x & 63) >> 4;
    const uint32_t shift = 6u - 2u * (uint32_t) g;
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
        i32x4v codes;
#pragma unroll
        for (int d = 0; d < 4; ++d) codes[d] = (int32_t) ((b[tn][d] >> shift) & 0x03030303u);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) c[tm][tn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[tm], codes, c[tm][tn], 0, 0, 0);
    }
}

constexpr int GEMM_DEPTH = 4;       // k steps of loads in flight per wave

// SPLIT = 1: the four waves sit side by side along the rows, each over all
// of K. SPLIT = 4: the four waves share one output tile and take a quarter
// of the k steps each; their int32 partial sums meet in LDS (exact in any
// order) and wave 0 writes the tile -- four times the workgroups for the
// small token counts whose grid would otherwise be a few dozen.
template <int TM, int TN, int SPLIT>
__device__ __forceinline__ void gemm_block(const gemm_args &G) {
    __shared__ i32x4v part[SPLIT > 1 ? SPLIT - 1 : 1][TM][TN][64];
    const int lane = threadIdx.x & 63, g = lane >> 4, li = lane & 15;
    const uint32_t wave = __builtin_amdgcn_readfirstlane((uint32_t) threadIdx.x >> 6);
    const gemm_view V = gemm_pick(G);
    const uint32_t t0 = blockIdx.y * 16u * TM;
    const uint32_t n0 = (SPLIT > 1 ? V.tile : V.tile * 4u + wave) * 16u * TN;
    const uint32_t steps_all = G.k / 64u;
    const uint32_t s_begin = SPLIT > 1 ? steps_all * wave / SPLIT : 0u;
    const uint32_t s_end = SPLIT > 1 ? steps_all * (wave + 1) / SPLIT : steps_all;
    i32x4v c[TM][TN];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) c[tm][tn] = (i32x4v) { 0, 0, 0, 0 };
    }
    // a ring of GEMM_DEPTH steps: step s lives in slot s % GEMM_DEPTH and is
    // refilled with step s + GEMM_DEPTH (the last step again past the end)
    i32x4v a[GEMM_DEPTH][TM];
    u32x4 bw[GEMM_DEPTH][TN];
    const uint32_t last = s_end > s_begin ? s_end - 1 : s_begin;
#pragma unroll
    for (int i = 0; i < GEMM_DEPTH; ++i) gemm_load<TM, TN>(G, V, t0, n0, min(s_begin + (uint32_t) i, last), a[i], bw[i]);
    for (uint32_t s = s_begin; s < s_end; s += GEMM_DEPTH) {
#pragma unroll
        for (int i = 0; i < GEMM_DEPTH; ++i) {
            if (s + (uint32_t) i < s_end) gemm_mma<TM, TN>(a[i], bw[i], c);
            gemm_load<TM, TN>(G, V, t0, n0, min(s + (uint32_t) i + GEMM_DEPTH, last), a[i], bw[i]);
        }
    }
    if (SPLIT > 1) {
        if (wave > 0) {
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) part[wave - 1][tm][tn][lane] = c[tm][tn];
            }
        }
        __syncthreads();
        if (wave > 0) return;
#pragma unroll
        for (int w = 0; w < SPLIT - 1; ++w) {
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) c[tm][tn] += part[w][tm][tn][lane];
            }
        }
    }

    // epilogue (src/i2s_gemm.c:271-290): post = w_scale / act_scale per
    // token, (float)(dot - sum) * post
    const float ws = G_CAST(const float, V.w + (size_t) V.n_rows * (G.k >> 2))[vzero()];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t t = t0 + 16u * (uint32_t) tm + 4u * (uint32_t) g + (uint32_t) r;
            if (t >= G.m) continue;
            const act_t at = G.act != nullptr ? G.act[t] : act_t { 1.0f, 0 };
            const float post = ws / at.scale;
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                const uint32_t n = n0 + 16u * (uint32_t) tn + (uint32_t) li;
                if (n < V.n_rows) {
                    const int32_t d = c[tm][tn][r];
                    if (V.out_i != nullptr) G_CAST(int32_t, V.out_i)[(size_t) t * V.n_rows + n] = d;
                    if (V.out != nullptr) G_CAST(float, V.out)[(size_t) t * V.n_rows + n] = (float) (d - at.sum) * post;
                }
            }
        }
    }
}


// Large token counts (the prefill chunk): the workgroup stages its tile
// through LDS so that each byte of the token rows and of the packed weights
// enters it once, not once per wave. 128 tokens x 128 rows per workgroup,
// four waves of 64 x 64 (16 MFMAs per k step); K moves in chunks of 256
// through one LDS buffer, the next chunk's global loads in registers while
// the current one is multiplied. One buffer (45 KB) and about 160 registers
// let three workgroups share a CU, so that one workgroup's barriers and
// LDS stores overlap the others' MFMAs. LDS rows are padded (272 bytes per
// token, 80 per weight row) so that the 16-byte operand reads of a lane
// group spread over the banks. K must be a multiple of 256.
constexpr uint32_t GL_BM = 128, GL_BN = 128, GL_BK = 256;
constexpr uint32_t GL_QS = GL_BK + 16, GL_WS = GL_BK / 4 + 16;
constexpr int GL_QLOADS = (int) (GL_BM * GL_BK / 16 / 256);
constexpr int GL_WLOADS = (int) (GL_BN * GL_BK / 4 / 16 / 256);

template <int NB>
struct gl_shared {
    uint8_t q[NB][GL_BM * GL_QS];
    uint8_t w[NB][GL_BN * GL_WS];
};

// SINGLE: one LDS buffer (45 KB, about 250 registers: two workgroups per
// CU), the next chunk in registers while the current one is multiplied,
// then the buffer rewritten between two barriers -- for grids of more than
// one workgroup per CU, where the workgroups sharing a CU overlap each
// other's barriers. Otherwise two LDS buffers (90 KB, one workgroup per
// CU) and the global loads two chunks ahead, so that a lone workgroup's
// loads overlap its own MFMAs.
template <bool SINGLE>
__device__ __forceinline__ void gemm_lds_block(const gemm_args &G) {
    constexpr int NB = SINGLE ? 1 : 2;
    __shared__ __attribute__((aligned(16))) gl_shared<NB> S;
    const gemm_view V = gemm_pick(G);
    const uint32_t tid = threadIdx.x;
    const int lane = (int) (tid & 63), g = lane >> 4, li = lane & 15;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t t0 = blockIdx.y * GL_BM, n0 = V.tile * GL_BN;
    const uint32_t wt = (wave >> 1) * 64u, wn = (wave & 1u) * 64u;
    const uint32_t chunks = G.k / GL_BK, kb = G.k >> 2;
    auto gload = [&](uint32_t c, u32x4 (&q)[GL_QLOADS], u32x4 (&w)[GL_WLOADS]) {
        const uint32_t cc = min(c, chunks - 1);
#pragma unroll
        for (int u = 0; u < GL_QLOADS; ++u) {
            const uint32_t p = tid + 256u * (uint32_t) u, tok = p / 16u, off = (p % 16u) * 16u;
            const uint32_t t = min(t0 + tok, G.m - 1);
            q[u] = *G_CAST(const u32x4, G.q + (size_t) t * G.k + cc * GL_BK + off);
        }
#pragma unroll
        for (int u = 0; u < GL_WLOADS; ++u) {
            const uint32_t p = tid + 256u * (uint32_t) u, row = p / 4u, off = (p % 4u) * 16u;
            const uint32_t n = min(n0 + row, V.n_rows - 1);
            w[u] = __builtin_nontemporal_load(G_CAST(const u32x4, V.w + (size_t) n * kb + cc * (GL_BK / 4) + off));
        }
    };
    auto lstore = [&](int buf, const u32x4 (&q)[GL_QLOADS], const u32x4 (&w)[GL_WLOADS]) {
#pragma unroll
        for (int u = 0; u < GL_QLOADS; ++u) {
            const uint32_t p = tid + 256u * (uint32_t) u, tok = p / 16u, off = (p % 16u) * 16u;
            *reinterpret_cast<u32x4 *>(&S.q[buf][tok * GL_QS + off]) = q[u];
        }
#pragma unroll
        for (int u = 0; u < GL_WLOADS; ++u) {
            const uint32_t p = tid + 256u * (uint32_t) u, row = p / 4u, off = (p % 4u) * 16u;
            *reinterpret_cast<u32x4 *>(&S.w[buf][row * GL_WS + off]) = w[u];
        }
    };
    i32x4v c[4][4];
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) c[tm][tn] = (i32x4v) { 0, 0, 0, 0 };
    }
    const uint32_t shift = 6u - 2u * (uint32_t) g;
    auto compute = [&](int buf) {
#pragma unroll
        for (int ks = 0; ks < (int) (GL_BK / 64); ++ks) {
            const uint32_t blk = (uint32_t) ks >> 1, h = (uint32_t) ks & 1u;
            i32x4v a[4], b[4];
#pragma unroll
            for (int tm = 0; tm < 4; ++tm) {
                const uint32_t row = wt + 16u * (uint32_t) tm + (uint32_t) li;
                a[tm] = *reinterpret_cast<const i32x4v *>(&S.q[buf][row * GL_QS + 128u * blk + 32u * (uint32_t) g + 16u * h]);
            }
#pragma unroll
            for (int tn = 0; tn < 4; ++tn) {
                const uint32_t row = wn + 16u * (uint32_t) tn + (uint32_t) li;
                const u32x4 raw = *reinterpret_cast<const u32x4 *>(&S.w[buf][row * GL_WS + 32u * blk + 16u * h]);
#pragma unroll
                for (int d = 0; d < 4; ++d) b[tn][d] = (int32_t) ((raw[d] >> shift) & 0x03030303u);
            }
#pragma unroll
            for (int tm = 0; tm < 4; ++tm) {
#pragma unroll
                for (int tn = 0; tn < 4; ++tn) c[tm][tn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[tm], b[tn], c[tm][tn], 0, 0, 0);
            }
        }
    };
    if (SINGLE) {
        u32x4 qn[GL_QLOADS], wn_[GL_WLOADS];
        gload(0, qn, wn_);
        lstore(0, qn, wn_);
        __syncthreads();
        // chunk ch is multiplied from LDS while chunk ch + 1 arrives in
        // registers; then the buffer is rewritten between two barriers
        for (uint32_t ch = 0; ch < chunks; ++ch) {
            gload(ch + 1, qn, wn_);
            compute(0);
            if (ch + 1 >= chunks) break;          // uniform
            __syncthreads();
            lstore(0, qn, wn_);
            __syncthreads();
        }
    } else {
        u32x4 q0[GL_QLOADS], w0[GL_WLOADS], q1[GL_QLOADS], w1[GL_WLOADS];
        gload(0, q0, w0);
        gload(1, q1, w1);
        lstore(0, q0, w0);
        __syncthreads();
        // chunk ch computes from LDS buffer ch & 1; register set ch & 1 is
        // refilled with chunk ch + 2 while it runs
        for (uint32_t ch = 0; ch < chunks; ch += 2) {
            gload(ch + 2, q0, w0);
            compute(0);
            lstore(1, q1, w1);
            __syncthreads();
            if (ch + 1 >= chunks) break;
            gload(ch + 3, q1, w1);
            compute(1);
            lstore(0, q0, w0);
            __syncthreads();
        }
    }

    const float ws = G_CAST(const float, V.w + (size_t) V.n_rows * kb)[vzero()];
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t t = t0 + wt + 16u * (uint32_t) tm + 4u * (uint32_t) g + (uint32_t) r;
            if (t >= G.m) continue;
            const act_t at = G.act != nullptr ? G.act[t] : act_t { 1.0f, 0 };
            const float post = ws / at.scale;
#pragma unroll
            for (int tn = 0; tn < 4; ++tn) {
                const uint32_t n = n0 + wn + 16u * (uint32_t) tn + (uint32_t) li;
                if (n < V.n_rows) {
                    const int32_t d = c[tm][tn][r];
                    if (V.out_i != nullptr) G_CAST(int32_t, V.out_i)[(size_t) t * V.n_rows + n] = d;
                    if (V.out != nullptr) G_CAST(float, V.out)[(size_t) t * V.n_rows + n] = (float) (d - at.sum) * post;
                }
            }
        }
    }
}

// Direct-load tiles (K % 256 == 0). K moves in super-steps of 256: two I2_S
// blocks, 256 bytes of each token row and 64 packed bytes of each weight row.
// global_load_lds_dwordx4 copies both straight from global memory into a
// ring of STAGES LDS stages, STAGES - 1 super-steps ahead, with no registers
// or LDS stores in between; each wave waits on its own copies (vmcnt) and one
// barrier per super-step makes every wave's copies visible.
//
// Operand layout. Lane group g of a wave takes chunk g of its row's 64 packed
// bytes (block 2s + g/2, half g%2) and feeds fields f = 0..3 of it to four
// MFMA steps; its int8 operand for step f is the 16 token bytes at
// k = 256 s + 128 (g/2) + 32 f + 16 (g%2) -- the elements the field holds
// (block layout in the file header). So one 16-byte weight read serves four
// steps, and every dot still sums the same products as the reference's.
//
// LDS layout: a token row is 16 granules of 16 bytes, granule G of token t at
// slot G ^ (t % 16); a weight row is 4 chunks, chunk c of row r at slot
// c ^ ((r / 4) % 4). The 16 lanes of a lane group then read 16 distinct banks
// groups. The copies fill LDS in lane order, so each lane fetches the global
// granule that belongs at its slot.
//
// A workgroup is 16 TM tokens x 64 TN rows: four waves side by side along the
// rows, each 16 TM tokens x 16 TN rows (TM x TN MFMA tiles). Within a super-
// step the next step's operand reads and weight unpacking are interleaved
// with the current step's MFMAs, which keep the matrix unit busy while the
// SIMD issues them.
template <int N>
__device__ __forceinline__ void wait_vmem() {   // s_waitcnt vmcnt(N), the other counters untouched
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

#define LDS_PTR(p) ((__attribute__((address_space(3))) void *) (p))

// XCD-aware placement. Workgroups are dealt to the eight XCDs round-robin by
// linear id (x fastest); XCD s is given a contiguous run of the tiles, row
// tile slowest, so the workgroups that share a weight tile (all its token
// tiles) share one L2 and the weights cross the fabric once, not once per
// token tile. (bx, by): this workgroup's row tile and token tile.
__device__ __forceinline__ void gemm_place(uint32_t &bx, uint32_t &by) {
    const uint32_t gx = gridDim.x, gy = gridDim.y, n = gx * gy;
    const uint32_t lin = blockIdx.y * gx + blockIdx.x;
    const uint32_t s = lin & 7u, q = n >> 3, r = n & 7u;     // XCD s holds q + (s < r) workgroups
    const uint32_t t = s * q + min(s, r) + (lin >> 3);
    bx = t / gy;
    by = t - bx * gy;
}

// The end of a direct-load tile (src/i2s_gemm.c:271-290): post = w_scale /
// act_scale per token, then (float)(dot - sum) * post. Each K group writes
// its int32 sums to a tile of its own in LDS (S, at least KG BM (BN + 4) +
// 2 BM words) and the stores add the KG tiles up (exact in any order), so
// one barrier separates the writes from the stores and every wave takes
// part in both. The tile goes through LDS so that every store writes whole
// rows of the output: a lane's accumulators hold rows 16 apart, the store
// wants four consecutive ones per lane. The caller has drained its copies
// into S.
template <int TM, int TN, int KG, bool ROPE = false, bool GLU = false, bool RES = false>
__device__ __forceinline__ void gemm_tile_epilogue(uint8_t *S, const gemm_view &V, uint32_t m, uint32_t t0,
                                                   uint32_t n0, uint32_t wr, uint32_t kgrp, uint32_t wave_all,
                                                   float ep_ws, float ep_ws2, act_t ep_at, i32x4v (&c)[TM][TN],
                                                   const gemm_rope *R) {
    constexpr uint32_t BM = 16u * TM, BN = 64u * TN;
    constexpr uint32_t EP = BN + 4u, E_TILE = BM * EP * 4u;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t g = lane >> 4, li = lane & 15u;
    __syncthreads();                                // every wave done with the ring
    uint32_t *mine = reinterpret_cast<uint32_t *>(S + kgrp * E_TILE);
    float *post_s = reinterpret_cast<float *>(S + KG * E_TILE);
    int32_t *sum_s = reinterpret_cast<int32_t *>(S + KG * E_TILE + BM * 4u);
    float *post2_s = reinterpret_cast<float *>(S + KG * E_TILE + BM * 8u);   // GLU: the up tensor's
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                mine[(16u * (uint32_t) tm + 4u * g + (uint32_t) r) * EP + wr + 16u * (uint32_t) tn + li] =
                    (uint32_t) c[tm][tn][r];
    if (tid < BM) {
        post_s[tid] = ep_ws / ep_at.scale;
        sum_s[tid] = ep_at.sum;
        if (GLU) post2_s[tid] = ep_ws2 / ep_at.scale;
    }
    __syncthreads();
    const bool vec_f = (V.n_rows & 3u) == 0 && ((uintptr_t) V.out & 15u) == 0;
    // streaming stores: written through as the tiles finish rather than left
    // dirty in L2 for the end-of-kernel writeback
    auto put = [&](bool vec, GLOBAL uint32_t *o, uint32_t n, u32x4 v) {
        if (vec) {
            __builtin_nontemporal_store(v, reinterpret_cast<GLOBAL u32x4 *>(o));
        } else {
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e) if (n + e < V.n_rows) __builtin_nontemporal_store(v[e], o + e);
        }
    };
    if constexpr (GLU) {
        // columns [0, BN / 2) of the tile are gate rows n0 .., columns
        // [BN / 2, BN) the same rows of up: h = silu(gate) * up
        // (src/forward.c:776-778), each factor as the plain epilogue makes it
        constexpr uint32_t HB = BN / 2u, GLPT = HB / 4u, GRPS = 64u / GLPT;
        const uint32_t grow = lane / GLPT, gcol = 4u * (lane % GLPT);
        for (uint32_t row0 = wave_all * GRPS; row0 < BM; row0 += 4u * KG * GRPS) {
            const uint32_t row = row0 + grow, t = t0 + row, n = n0 + gcol;
            if (t < m && n < V.n_rows) {
                i32x4v dg = *reinterpret_cast<const i32x4v *>(S + (row * EP + gcol) * 4u);
                i32x4v du = *reinterpret_cast<const i32x4v *>(S + (row * EP + HB + gcol) * 4u);
#pragma unroll
                for (uint32_t k2 = 1; k2 < (uint32_t) KG; ++k2) {
                    dg += *reinterpret_cast<const i32x4v *>(S + k2 * E_TILE + (row * EP + gcol) * 4u);
                    du += *reinterpret_cast<const i32x4v *>(S + k2 * E_TILE + (row * EP + HB + gcol) * 4u);
                }
                const float pg = post_s[row], pu = post2_s[row];
                const int32_t sum = sum_s[row];
                u32x4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float gf = (float) (dg[e] - sum) * pg, uf = (float) (du[e] - sum) * pu;
                    v[e] = __float_as_uint(silu(gf) * uf);
                }
                put(vec_f, G_CAST(uint32_t, V.out) + (size_t) t * V.n_rows + n, n, v);
            }
        }
        return;
    }
    constexpr uint32_t LPT = BN / 4u;               // lanes per tile row in the stores
    constexpr uint32_t RPS = 64u / LPT;             // tile rows per store instruction
    const uint32_t srow = lane / LPT, scol = 4u * (lane % LPT);
    if constexpr (ROPE) {
        // the tile's rows are whole heads of one job (n0 and BN multiples of
        // hd): values go straight to the value cache; query and key floats
        // go back into LDS (over K group 0's tile) so that each dimension
        // finds its rotary partner, then out to the q rows / the key cache
        constexpr uint32_t NP = BM / (4u * KG * RPS);  // rows of this lane
        const uint32_t hd = R->hd, half = R->half;
        const uint32_t dd = (n0 + scol) % hd;          // the lane's first dimension (of four)
        const uint32_t e0 = dd < half ? dd : (dd < 2u * half ? dd - half : 0u);
        float fr[NP][4];
        f32x4 csa[NP][2];                              // (cos, sin) of dimensions dd .. dd + 3
#pragma unroll
        for (uint32_t p = 0; p < NP; ++p) {
            const uint32_t row = wave_all * RPS + p * 4u * KG * RPS + srow, t = t0 + row, n = n0 + scol;
            const GLOBAL float *cs = G_CAST(const float, R->rope) +
                                     ((size_t) (R->pos0 + min(t, m - 1)) * half + e0) * 2u;
            csa[p][0] = *reinterpret_cast<const GLOBAL f32x4 *>(cs);
            csa[p][1] = *reinterpret_cast<const GLOBAL f32x4 *>(cs + 4);
            i32x4v d = *reinterpret_cast<const i32x4v *>(S + (row * EP + scol) * 4u);
#pragma unroll
            for (uint32_t k2 = 1; k2 < (uint32_t) KG; ++k2)
                d += *reinterpret_cast<const i32x4v *>(S + k2 * E_TILE + (row * EP + scol) * 4u);
            const float post = post_s[row];
            const int32_t sum = sum_s[row];
#pragma unroll
            for (int e = 0; e < 4; ++e) fr[p][e] = (float) (d[e] - sum) * post;
            if (V.job == 2 && t < m && n < V.n_rows) {
                // slice-major (both caches): [KV head][dimension / 8][position][dimension % 8]
                GLOBAL float *o = G_CAST(float, R->v_cache) +
                                  (((size_t) (n / hd) * (hd / 8u) + dd / 8u) * R->n_ctx + R->pos0 + t) * 8u + dd % 8u;
                *reinterpret_cast<GLOBAL f32x4 *>(o) = (f32x4) { fr[p][0], fr[p][1], fr[p][2], fr[p][3] };
            }
        }
        if (V.job == 2) return;                         // uniform
        __syncthreads();                                // every read of the int32 tiles done
        float *F = reinterpret_cast<float *>(S);
#pragma unroll
        for (uint32_t p = 0; p < NP; ++p) {
            const uint32_t row = wave_all * RPS + p * 4u * KG * RPS + srow;
            *reinterpret_cast<f32x4 *>(F + row * EP + scol) = (f32x4) { fr[p][0], fr[p][1], fr[p][2], fr[p][3] };
        }
        __syncthreads();
#pragma unroll
        for (uint32_t p = 0; p < NP; ++p) {
            const uint32_t row = wave_all * RPS + p * 4u * KG * RPS + srow, t = t0 + row, n = n0 + scol;
            if (t < m && n < V.n_rows) {
                f32x4 o;
#pragma unroll
                for (uint32_t e = 0; e < 4u; ++e) {
                    const uint32_t de = dd + e, col = scol + e, hb = col - de;
                    const uint32_t partner = de < half ? de + half : (de < 2u * half ? de - half : de);
                    const float x = F[row * EP + col], y = F[row * EP + hb + partner];
                    const float cc = csa[p][e / 2u][2u * (e % 2u)], ss = csa[p][e / 2u][2u * (e % 2u) + 1u];
                    o[e] = de < half ? x * cc - y * ss : (de < 2u * half ? y * ss + x * cc : x);
                }
                GLOBAL float *dst = V.job == 0
                    ? G_CAST(float, V.out) + (size_t) t * V.n_rows + n
                    : G_CAST(float, R->k_cache) +
                          (((size_t) (n / hd) * (hd / 8u) + dd / 8u) * R->n_ctx + R->pos0 + t) * 8u + dd % 8u;
                *reinterpret_cast<GLOBAL f32x4 *>(dst) = o;
            }
        }
        return;
    }
    const bool vec_i = (V.n_rows & 3u) == 0 && ((uintptr_t) V.out_i & 15u) == 0;
    const bool vec_r = vec_f && ((uintptr_t) V.res & 15u) == 0;
    for (uint32_t row0 = wave_all * RPS; row0 < BM; row0 += 4u * KG * RPS) {
        const uint32_t row = row0 + srow, t = t0 + row, n = n0 + scol;
        if (t < m && n < V.n_rows) {
            i32x4v d = *reinterpret_cast<const i32x4v *>(S + (row * EP + scol) * 4u);
#pragma unroll
            for (uint32_t k2 = 1; k2 < (uint32_t) KG; ++k2)
                d += *reinterpret_cast<const i32x4v *>(S + k2 * E_TILE + (row * EP + scol) * 4u);
            const size_t at = (size_t) t * V.n_rows + n;
            if (V.out_i != nullptr) put(vec_i, G_CAST(uint32_t, V.out_i) + at, n, (u32x4) d);
            if (V.out != nullptr) {
                const float post = post_s[row];
                const int32_t sum = sum_s[row];
                u32x4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = __float_as_uint((float) (d[e] - sum) * post);
                if (RES) {
                    // the residual sums (src/forward.c:744-750, :795-800): out + res
                    if (vec_r) {
                        const f32x4 r = *reinterpret_cast<const GLOBAL f32x4 *>(G_CAST(const float, V.res) + at);
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = __float_as_uint(__uint_as_float(v[e]) + r[e]);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (n + (uint32_t) e < V.n_rows) v[e] = __float_as_uint(__uint_as_float(v[e]) + V.res[at + e]);
                    }
                }
                put(vec_f, G_CAST(uint32_t, V.out) + at, n, v);
            }
        }
    }
}

// KG K groups: with KG = 2 the workgroup is eight waves, two groups of four
// over the same tile; group k takes super-steps k, k + 2, k + 4, ... (two
// waves on every SIMD, one of each group, so that one's waits are covered by
// the other's MFMAs), and the groups' int32 sums meet in LDS at the end
// (exact in any order).
// GLU: a gate + up tile (V.w gate, V.w2 up, n_rows each): BN / 2 rows of
// each tensor, gate's in K group 0's half of the weight slot and up's in
// group 1's, so that the epilogue finds both factors of every output.
template <int TM, int TN, int STAGES, int KG = 1, bool ROPE = false, bool GLU = false, bool RES = false>
__device__ __forceinline__ void gemm_dl_tile(const gemm_view &V, uint32_t k, uint32_t m, uint32_t by,
                                             const gemm_rope *R = nullptr) {
    constexpr uint32_t BM = 16u * TM, BN = 64u * TN;
    constexpr uint32_t A_BYTES = BM * 256u, STAGE = A_BYTES + BN * 64u;
    constexpr int VM = TM + TN;                     // copies per wave per super-step
    constexpr int D = STAGES / KG;                  // ring depth in iterations
    static_assert(KG == 1 || KG == 2 || KG == 4, "K groups");
    static_assert(STAGES % KG == 0 && D >= 2 && (D - 2) * VM < 64, "stages");
    // WL (with K groups): the weights of a whole iteration (KG super-steps,
    // PB bytes of each row) arrive together, 8 rows x 128 bytes or 4 rows x
    // 256 bytes per copy instruction, whole cache lines where the row is
    // line-aligned -- 16 rows x 64 bytes per instruction streams at about
    // 5.1 TB/s on MI355X against 6.0-6.9 for whole lines. LDS then holds
    // STAGES token slots, then D weight slots of BN rows x PB bytes (the
    // same total); chunk c of row r of a weight slot sits at slot c ^ (r % 8).
    constexpr bool WL = KG >= 2;
    constexpr uint32_t PB = 64u * KG, CR = 4u * KG, A_REGION = STAGES * A_BYTES, WSLOT = BN * PB;
    // the epilogue reuses the ring: KG tiles of BM rows of EP (BN + 4) words,
    // then post and sum of the BM tokens
    constexpr uint32_t EP = BN + 4u, E_TILE = BM * EP * 4u, E_BYTES = KG * E_TILE + BM * (GLU ? 12u : 8u);
    constexpr uint32_t S_BYTES = STAGES * STAGE > E_BYTES ? STAGES * STAGE : E_BYTES;
    __shared__ __attribute__((aligned(1024))) uint8_t S[S_BYTES];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave_all = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wave = wave_all & 3u, kgrp = wave_all >> 2;   // place in the tile, K group
    const uint32_t g = lane >> 4, li = lane & 15u;
    static_assert(!GLU || KG == 2, "a gate + up tile is two K groups, one per tensor");
    const uint32_t t0 = by * BM, n0 = V.tile * (GLU ? BN / 2u : BN);
    const uint32_t nsup = k / 256u, kb = k >> 2;
    // the epilogue's operands, loaded now so that their latency hides behind
    // the main loop: w_scale, and token t0 + tid's act for the first BM threads
    float ep_ws = 0.0f, ep_ws2 = 0.0f;
    act_t ep_at = { 1.0f, 0 };
    if (tid < BM) {
        // the sixteen-wave tiles (a few tokens, one token tile): a vector
        // load, so that the first wait on the scalar loads does not stall on
        // it; the others (weight tiles shared in L2 by several token tiles)
        // measured faster with the scalar load
        const GLOBAL float *wsp = G_CAST(const float, V.w + (size_t) V.n_rows * kb);
        if (KG == 4) ep_ws = wsp[vzero()];
        else ep_ws = *wsp;
        if (GLU) ep_ws2 = *G_CAST(const float, V.w2 + (size_t) V.n_rows * kb);
        if (V.act != nullptr) ep_at = V.act[min(t0 + tid, m - 1)];
    }
    // copy sources: instruction j of this wave fills LDS granules
    // (4 j + wave) * 64 + lane of the token and the weight block
    const int8_t *asrc[TM];
#pragma unroll
    for (int j = 0; j < TM; ++j) {
        const uint32_t p = ((uint32_t) j * 4u + wave) * 64u + lane;
        const uint32_t t = p >> 4, gr = (p & 15u) ^ (t & 15u);
        asrc[j] = V.q + (size_t) min(t0 + t, m - 1) * k + gr * 16u;
    }
    const uint8_t *bsrc[TN];
    uint32_t bch[TN];                               // WL: the chunk (of CR) each copy lane fetches
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const uint32_t p = ((uint32_t) j * 4u + wave) * 64u + lane;
        if (WL) {                                   // K group kgrp copies rows [kgrp BN/KG, (kgrp + 1) BN/KG)
            const uint32_t r = kgrp * (BN / KG) + p / CR;
            bch[j] = (p % CR) ^ (r & 7u);
            if (GLU) bsrc[j] = (kgrp == 0 ? V.w : V.w2) + (size_t) min(n0 + r - kgrp * (BN / 2u), V.n_rows - 1) * kb;
            else bsrc[j] = V.w + (size_t) min(n0 + r, V.n_rows - 1) * kb;
        } else {
            const uint32_t r = p >> 2, ch = (p & 3u) ^ ((r >> 2) & 3u);
            bch[j] = 0;
            bsrc[j] = V.w + (size_t) min(n0 + r, V.n_rows - 1) * kb + ch * 16u;
        }
    }
    const uint32_t iters = (nsup + KG - 1) / KG;
    // super-step s lives in slot s % STAGES (WL: its tokens; its iteration's
    // weights in weight slot (s / KG) % D); past the end the last one is
    // copied again (never read), and a WL chunk past the last super-step
    // copies the iteration's first super-step's instead
    auto issue = [&](uint32_t s) {
        const uint32_t sc = min(s, nsup - 1);
        uint8_t *base = S + (s % STAGES) * (WL ? A_BYTES : STAGE);
#pragma unroll
        for (int j = 0; j < TM; ++j)
            __builtin_amdgcn_global_load_lds((const void *) (asrc[j] + sc * 256u),
                                             LDS_PTR(base + ((uint32_t) j * 4u + wave) * 1024u), 16, 0, 0);
        if (WL) {
            const uint32_t it = min(s / KG, iters - 1);
            uint8_t *wbase = S + A_REGION + ((s / KG) % D) * WSLOT + kgrp * (BN / KG) * PB;
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const uint32_t ch = KG * it + bch[j] / 4u < nsup ? bch[j] : (bch[j] & 3u);
                __builtin_amdgcn_global_load_lds((const void *) (bsrc[j] + it * PB + ch * 16u),
                                                 LDS_PTR(wbase + ((uint32_t) j * 4u + wave) * 1024u), 16, 0, 0);
            }
        } else {
#pragma unroll
            for (int j = 0; j < TN; ++j)
                __builtin_amdgcn_global_load_lds((const void *) (bsrc[j] + sc * 64u),
                                                 LDS_PTR(base + A_BYTES + ((uint32_t) j * 4u + wave) * 1024u), 16, 0, 0);
        }
    };
    uint32_t aoff[4];                               // token 16 tm + li (tm * 4096 added), granule of step f
#pragma unroll
    for (int f = 0; f < 4; ++f) aoff[f] = li * 256u + (((8u * (g >> 1) + 2u * (uint32_t) f + (g & 1u)) ^ li) * 16u);
    const uint32_t wr = wave * (16u * TN);          // this wave's first row in the tile
    // this lane's weight chunk: row wr + li (+ 16 tn), chunk g of the super-step
    const uint32_t boff = WL ? A_REGION + (wr + li) * PB + (((4u * kgrp + g) ^ (li & 7u)) * 16u)
                             : A_BYTES + (wr + li) * 64u + ((g ^ ((li >> 2) & 3u)) * 16u);
    constexpr uint32_t BROW16 = WL ? 16u * PB : 1024u;   // 16 rows further
    i32x4v c[TM][TN];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) c[tm][tn] = (i32x4v) { 0, 0, 0, 0 };
    }
    // iteration it: group k multiplies super-step KG it + k
#pragma unroll
    for (int i = 0; i < D - 1; ++i) issue((uint32_t) (KG * i) + kgrp);
    for (uint32_t it = 0; it < iters; ++it) {
        const uint32_t s = KG * it + kgrp;
        // this iteration's copies done (later ones may stay in flight), then everyone's
        // (near the end, fewer are in flight: wait for all but the next one)
        const uint32_t ahead = min(iters - 1u - it, (uint32_t) D - 2u);
        if (ahead == (uint32_t) D - 2u) wait_vmem<(D - 2) * VM>();
        else if (ahead == 1) wait_vmem<VM>();
        else wait_vmem<0>();
        __builtin_amdgcn_s_waitcnt(0xC07F);         // lgkmcnt(0): this wave's reads of the stage being refilled done
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        issue(s + (uint32_t) (KG * (D - 1)));
        __builtin_amdgcn_sched_barrier(0);
        if (KG > 1 && s >= nsup) continue;          // an odd count: the last iteration is group 0's alone
        const uint8_t *st = S + (s % STAGES) * (WL ? A_BYTES : STAGE);
        const uint8_t *sw = WL ? S + (it % D) * WSLOT : st;
        u32x4 raw[TN];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) raw[tn] = *reinterpret_cast<const u32x4 *>(sw + boff + (uint32_t) tn * BROW16);
        i32x4v a[2][TM], b[2][TN];
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) a[0][tm] = *reinterpret_cast<const i32x4v *>(st + aoff[0] + (uint32_t) tm * 4096u);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
#pragma unroll
            for (int d = 0; d < 4; ++d) b[0][tn][d] = (int32_t) ((raw[tn][d] >> 6u) & 0x03030303u);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int f = 0; f < 4; ++f) {
            const int cu = f & 1, nx = cu ^ 1;
            if (f < 3) {
#pragma unroll
                for (int tm = 0; tm < TM; ++tm)
                    a[nx][tm] = *reinterpret_cast<const i32x4v *>(st + aoff[f + 1] + (uint32_t) tm * 4096u);
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) {
#pragma unroll
                    for (int d = 0; d < 4; ++d) b[nx][tn][d] = (int32_t) ((raw[tn][d] >> (4u - 2u * (uint32_t) f)) & 0x03030303u);
                }
            }
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
#pragma unroll
                for (int tm = 0; tm < TM; ++tm)
                    c[tm][tn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[cu][tm], b[cu][tn], c[tm][tn], 0, 0, 0);
            }
            if (f < 3) {
                // each MFMA, then one of the next step's reads and its share of the unpacking
                constexpr int VPM = (8 * TN + TM * TN - 1) / (TM * TN);
#pragma unroll
                for (int i = 0; i < TM * TN; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if (i < TM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    wait_vmem<0>();                                 // no copy may land after the workgroup leaves
    gemm_tile_epilogue<TM, TN, KG, ROPE, GLU, RES>(S, V, m, t0, n0, wr, kgrp, wave_all, ep_ws, ep_ws2, ep_at, c, R);
}

// the tile of a three-job launch (gemm_args) or of a plan (gemm_table)
template <int TM, int TN, int STAGES, int KG = 1, bool ROPE = false>
__device__ __forceinline__ void gemm_dl_block(const gemm_args &G, const gemm_rope *R = nullptr) {
    uint32_t bx, by;
    gemm_place(bx, by);
    gemm_dl_tile<TM, TN, STAGES, KG, ROPE>(gemm_pick(G, bx), G.k, G.m, by, R);
}

// a gate + up launch: job 0 of gemm_args is gate, job 1 up (the same
// n_rows); tiles[0] counts the row tiles of BN / 2 rows of each
template <int TM, int TN, int STAGES>
__device__ __forceinline__ void gemm_dl_glu(const gemm_args &G) {
    uint32_t bx, by;
    gemm_place(bx, by);
    const gemm_view V = { G.w[0], G.out[0], nullptr, G.n_rows[0], bx, G.q, G.act, 0u, G.w[1] };
    gemm_dl_tile<TM, TN, STAGES, 2, false, true>(V, G.k, G.m, by);
}

// one tensor (job 0 of gemm_args) whose f32 output gets a residual added:
// out = (dot - sum) * post + res, res of the output's shape
template <int TM, int TN, int STAGES, int KG>
__device__ __forceinline__ void gemm_dl_res(const gemm_args &G, const float *res) {
    uint32_t bx, by;
    gemm_place(bx, by);
    gemm_view V = gemm_pick(G, bx);
    V.res = res;
    gemm_dl_tile<TM, TN, STAGES, KG, false, false, true>(V, G.k, G.m, by);
}

template <int TM, int TN, int STAGES, int KG = 1>
__device__ __forceinline__ void gemm_dl_table(const gemm_table &T) {
    uint32_t bx, by;
    gemm_place(bx, by);
    const gemm_tjob &J = T.jobs[T.tile_job[bx]];
    const gemm_view V = { J.w, J.out, J.out_i, J.n_rows, bx - J.tile0, J.q, J.act, 0u };
    gemm_dl_tile<TM, TN, STAGES, KG>(V, J.k, T.m, by);
}

// ---------------------------------------------------------------------------
// GEMM plans of a few tokens as one stream per workgroup
// ---------------------------------------------------------------------------
//
// A plan's row tiles (128 rows of one tensor each) are cut into contiguous
// runs of about equal weight bytes, one run per workgroup (with several
// token tiles, one workgroup per run and token tile). The workgroup streams
// its run through one ring of LDS stages, as the direct-load tiles do, but
// the ring does not stop at a tile's end: the copies run D - 1 iterations
// ahead across tile boundaries, so a tile's start never waits for memory
// and its epilogue runs while the next tile's copies are in flight. Each
// tile's sums go to one of two LDS tiles at its last iteration and are
// stored at the next one. The stores are buffer stores, always issued
// (lanes with nothing to store aim past the buffer), so that every wave
// knows how many vector memory instructions it has issued, and each wait
// for an iteration's copies names exactly the instructions issued after
// them (loads and stores complete in order).

// One row tile of a streamed plan (mirrored in gfx950_shim.c).
struct gemm_srec {
    const uint8_t *w;          // the tile's first weight row; rows past `rows` clamp to its last
    const int8_t  *q;          // the job's int8 token rows [m][k]
    float         *out;        // the job's [m][n_rows] epilogue from the tile's first column, or null
    int32_t       *out_i;      // raw dots from the tile's first column, or null
    const act_t   *act;        // [m], or null without an epilogue
    const float   *ws;         // the tensor's w_scale
    uint32_t       k, rows, n_rows, vec;   // vec: float4 stores (n_rows % 4 == 0, outputs 16-byte aligned)
};
static_assert(sizeof(gemm_srec) == 64, "gemm_srec must match gfx950_shim.c");

struct gemm_stream {
    const gemm_srec *recs;     // every tile of the plan, in stream order
    const uint32_t  *range;    // [n_ranges + 1]: run r is recs[range[r] .. range[r + 1])
    uint32_t         m, gy, n_ranges, pad;
};
static_assert(sizeof(gemm_stream) == 32, "gemm_stream must match gfx950_shim.c");

constexpr uint32_t GS_RMAX = 64;       // tiles per run (the host cuts longer runs)
constexpr int GS_THREADS = 512;        // two K groups of four waves

// s_waitcnt vmcnt(n) for a uniform n (clamped to 63): a binary search over
// the immediates
template <int LO, int HI>
__device__ __forceinline__ void wait_vmem_rt(uint32_t n) {
    if constexpr (LO == HI) {
        wait_vmem<LO>();
    } else {
        constexpr int MID = (LO + HI) / 2;
        if (n <= (uint32_t) MID) wait_vmem_rt<LO, MID>(n);
        else wait_vmem_rt<MID + 1, HI>(n);
    }
}

template <typename T>
__device__ __forceinline__ T *uniform_ptr(T *p) {
    const uint64_t v = (uint64_t) (uintptr_t) p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t) v), hi = __builtin_amdgcn_readfirstlane((uint32_t) (v >> 32));
    return (T *) (uintptr_t) (((uint64_t) hi << 32) | lo);
}

// 16 tokens x 128 rows per tile; an iteration is two super-steps, one per
// K group (128 bytes of each weight row); D iterations in the ring.
// (Measured slower on the 96 FFN tensors: 64-row tiles reading 256 bytes of
// each row per iteration, and 32 x 128 tiles with a shallower ring.)
template <int D>
__device__ __forceinline__ void gemm_stream_body(const gemm_stream &P) {
    constexpr int TM = 1, TN = 2, SPG = 1;
    constexpr int KG = 2, SS = KG * SPG;           // super-steps per iteration
    constexpr uint32_t BM = 16u * TM, BN = 64u * TN;
    constexpr uint32_t A_BYTES = BM * 256u, PB = 64u * SS, CR = 4u * SS, WSLOT = BN * PB;
    constexpr int VM = (TM + TN) * SPG;            // copies per wave per iteration (and one more at a tile's first)
    static_assert(D >= 2 && D * (VM + 1) + 8 * TM < 64, "ring");
    constexpr uint32_t A_REGION = (uint32_t) (SS * D) * A_BYTES, W_REGION = D * WSLOT;
    constexpr uint32_t EP = BN + 4u, E_TILE = BM * EP * 4u, E_SET = KG * E_TILE;
    constexpr uint32_t EPS = 8u, EP_SLOT = 512u;   // a tile's act dwords, then w_scale at dword 127
    static_assert(2u * BM < 127u && EPS > (uint32_t) D, "tile constants");
    constexpr uint32_t OFF_E = A_REGION + W_REGION, OFF_EPS = OFF_E + 2u * E_SET, OFF_REC = OFF_EPS + EPS * EP_SLOT;
    constexpr uint32_t S_BYTES = OFF_REC + GS_RMAX * (uint32_t) sizeof(gemm_srec);
    static_assert(S_BYTES <= 160u * 1024u, "LDS");
    __shared__ __attribute__((aligned(1024))) uint8_t S[S_BYTES];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave_all = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wave = wave_all & 3u, kgrp = wave_all >> 2;
    const uint32_t g = lane >> 4, li = lane & 15u;

    // workgroup -> (token tile, run): the token tiles of one run on one XCD
    const uint32_t xcd = blockIdx.x & 7u, a8 = blockIdx.x >> 3;
    const uint32_t by = a8 % P.gy, run = (a8 / P.gy) * 8u + xcd;
    if (run >= P.n_ranges) return;                 // uniform
    const uint32_t r0 = P.range[run], nt = min(P.range[run + 1] - r0, GS_RMAX);
    if (nt == 0) return;
    gemm_srec *R = reinterpret_cast<gemm_srec *>(S + OFF_REC);
    for (uint32_t i = tid; i < nt * 4u; i += (uint32_t) GS_THREADS)
        reinterpret_cast<u32x4 *>(R)[i] = G_CAST(const u32x4, P.recs + r0)[i];
    __syncthreads();
    // the run's iterations, from its tiles' K: lane i takes tile i (nt <= 64)
    const uint32_t total = (uint32_t) wave_sum(lane < nt ? (int) ((R[lane].k / 256u + SS - 1) / SS) : 0);

    const uint32_t m = P.m, t0 = by * BM;
    // copy lanes: token row and (swizzled) granule of copy j; weight row and chunk
    constexpr int NB = TN * SPG;                   // weight copies per wave per iteration
    uint32_t a_t[TM], a_g[TM], b_r[NB], bch[NB];
#pragma unroll
    for (int j = 0; j < TM; ++j) {
        const uint32_t p = ((uint32_t) j * 4u + wave) * 64u + lane;
        a_t[j] = p >> 4;
        a_g[j] = (p & 15u) ^ (a_t[j] & 15u);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const uint32_t p = ((uint32_t) j * 4u + wave) * 64u + lane;
        b_r[j] = kgrp * (BN / KG) + p / CR;
        bch[j] = (p % CR) ^ (b_r[j] & 7u);
    }

    // the producer: tile pt, its iteration pit
    const int8_t *asrc[TM];
    const uint8_t *bsrc[NB];
    const uint32_t *epsrc = nullptr;
    uint32_t pt = 0, pit = 0, p_iters = 1, p_nsup = 1, gp = 0, ops = 0;
    auto p_enter = [&](uint32_t t) {
        const gemm_srec &rc = R[t];
        const uint32_t k = __builtin_amdgcn_readfirstlane(rc.k), kb = k >> 2;
        const uint32_t rows = __builtin_amdgcn_readfirstlane(rc.rows);
        const int8_t *q = uniform_ptr(rc.q);
        const uint8_t *w = uniform_ptr(rc.w);
        const act_t *act = uniform_ptr(rc.act);
        const float *ws = uniform_ptr(rc.ws);
        p_nsup = k / 256u;
        p_iters = (p_nsup + SS - 1) / SS;
#pragma unroll
        for (int j = 0; j < TM; ++j) asrc[j] = q + (size_t) min(t0 + a_t[j], m - 1) * k + a_g[j] * 16u;
#pragma unroll
        for (int j = 0; j < NB; ++j) bsrc[j] = w + (size_t) min(b_r[j], rows - 1) * kb;
        const uint32_t d = 64u * (wave & 1u) + lane;
        epsrc = act != nullptr && d < 2u * BM
            ? reinterpret_cast<const uint32_t *>(act + min(t0 + d / 2u, m - 1)) + (d & 1u)
            : reinterpret_cast<const uint32_t *>(ws);
    };
    // the producer's next iteration: each K group its super-step's tokens and
    // its half of the iteration's weight rows (whole lines: 8 rows x 128
    // bytes per instruction); at a tile's first iteration also the tile's
    // act and w_scale, one dword per lane
    auto issue = [&]() {
        const uint32_t slot = gp % (uint32_t) D;
#pragma unroll
        for (int u = 0; u < SPG; ++u) {
            const uint32_t l = SPG * kgrp + (uint32_t) u, s = min(SS * pit + l, p_nsup - 1);
            uint8_t *abase = S + (SS * slot + l) * A_BYTES;
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                // four token rows per copy; none past the last token (their
                // sums are never stored, whatever the slot holds)
                if (((uint32_t) j * 4u + wave) * 4u < m - t0) {        // uniform per wave
                    __builtin_amdgcn_global_load_lds((const void *) (asrc[j] + s * 256u),
                                                     LDS_PTR(abase + ((uint32_t) j * 4u + wave) * 1024u), 16, 0, 0);
                    ops += 1u;
                }
            }
        }
        uint8_t *wbase = S + A_REGION + slot * WSLOT + kgrp * (BN / KG) * PB;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const uint32_t ch = SS * pit + bch[j] / 4u < p_nsup ? bch[j] : (bch[j] & 3u);
            __builtin_amdgcn_global_load_lds((const void *) (bsrc[j] + pit * PB + ch * 16u),
                                             LDS_PTR(wbase + ((uint32_t) j * 4u + wave) * 1024u), 16, 0, 0);
        }
        ops += (uint32_t) NB;
        if (pit == 0) {                            // uniform
            __builtin_amdgcn_global_load_lds((const void *) epsrc,
                                             LDS_PTR(S + OFF_EPS + (pt % EPS) * EP_SLOT + (wave & 1u) * 256u), 4, 0, 0);
            ops += 1u;
        }
        ++gp;
        if (++pit == p_iters) {
            pit = 0;
            if (++pt < nt) p_enter(pt);
        }
    };

    // the stores of tile u, whose sums are in E set u % 2 (rows of 32 lanes x
    // four columns, two rows per instruction): (float)(dot - sum) * (w_scale /
    // act_scale), src/i2s_gemm.c:271-290
    auto store_tile = [&](uint32_t u) {
        const gemm_srec &rc = R[u];
        float *out = uniform_ptr(rc.out);
        int32_t *out_i = uniform_ptr(rc.out_i);
        const uint32_t rows = __builtin_amdgcn_readfirstlane(rc.rows), n_rows = __builtin_amdgcn_readfirstlane(rc.n_rows);
        const bool vec = __builtin_amdgcn_readfirstlane(rc.vec) != 0u;
        const uint32_t *cst = reinterpret_cast<const uint32_t *>(S + OFF_EPS + (u % EPS) * EP_SLOT);
        const float ws = __uint_as_float(cst[127]);
        const uint8_t *E0 = S + OFF_E + (u & 1u) * E_SET;
        const uint32_t limit = ((m - 1u) * n_rows + rows) * 4u;     // bytes from the tile's first column
        constexpr uint32_t LPT = BN / 4u, RPS = 64u / LPT;
        const uint32_t srow = lane / LPT, scol = 4u * (lane % LPT);
        const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(out, (short) 0, (int) limit, 0x00020000);
        const __amdgpu_buffer_rsrc_t ri = __builtin_amdgcn_make_buffer_rsrc(out_i, (short) 0, (int) limit, 0x00020000);
        for (uint32_t row0 = wave_all * RPS; row0 < BM; row0 += 8u * RPS) {    // uniform per wave
            const uint32_t row = row0 + srow, t = t0 + row;
            i32x4v d = *reinterpret_cast<const i32x4v *>(E0 + (row * EP + scol) * 4u);
            d += *reinterpret_cast<const i32x4v *>(E0 + E_TILE + (row * EP + scol) * 4u);
            const bool ok = t < m && scol < rows;
            const uint32_t at = ok ? (t * n_rows + scol) * 4u : 0xFFFFFFF0u;
            if (out_i != nullptr) {                // uniform
                if (vec) {
                    __builtin_amdgcn_raw_buffer_store_b128((u32x4) d, ri, (int) at, 0, CPOL_NT);
                    ops += 1u;
                } else {
#pragma unroll
                    for (uint32_t e = 0; e < 4u; ++e) {
                        const uint32_t ae = ok && scol + e < rows ? at + 4u * e : 0xFFFFFFF0u;
                        __builtin_amdgcn_raw_buffer_store_b32((uint32_t) d[e], ri, (int) ae, 0, CPOL_NT);
                    }
                    ops += 4u;
                }
            }
            if (out != nullptr) {                  // uniform
                const float sc = __uint_as_float(cst[2u * row]);
                const int32_t sum = (int32_t) cst[2u * row + 1u];
                const float post = ws / sc;
                u32x4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = __float_as_uint((float) (d[e] - sum) * post);
                if (vec) {
                    __builtin_amdgcn_raw_buffer_store_b128(v, ro, (int) at, 0, CPOL_NT);
                    ops += 1u;
                } else {
#pragma unroll
                    for (uint32_t e = 0; e < 4u; ++e) {
                        const uint32_t ae = ok && scol + e < rows ? at + 4u * e : 0xFFFFFFF0u;
                        __builtin_amdgcn_raw_buffer_store_b32(v[e], ro, (int) ae, 0, CPOL_NT);
                    }
                    ops += 4u;
                }
            }
        }
    };

    uint32_t aoff[4];                              // token 16 tm + li (tm * 4096 added), granule of step f
#pragma unroll
    for (int f = 0; f < 4; ++f) aoff[f] = li * 256u + (((8u * (g >> 1) + 2u * (uint32_t) f + (g & 1u)) ^ li) * 16u);
    const uint32_t wr = wave * (16u * TN);         // this wave's first row in the tile
    constexpr uint32_t BROW16 = 16u * PB;
    i32x4v c[TM][TN];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) c[tm][tn] = (i32x4v) { 0, 0, 0, 0 };

    p_enter(0);
    uint32_t mk[D - 1];                            // ops issued up to iteration G + i's copies
#pragma unroll
    for (int i = 0; i < D - 1; ++i) {
        if (gp < total) issue();
        mk[i] = ops;
    }
    uint32_t ct = 0, cit = 0;
    uint32_t c_nsup = __builtin_amdgcn_readfirstlane(R[0].k) / 256u, c_iters = (c_nsup + SS - 1) / SS;
    bool pend = false;                             // tile ct - 1's sums wait in E
    for (uint32_t G = 0; G < total; ++G) {
        wait_vmem_rt<0, 63>(min(ops - mk[0], 63u));   // this iteration's copies done
        __builtin_amdgcn_s_waitcnt(0xC07F);         // lgkmcnt(0): this wave's LDS reads and writes done
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (gp < total) issue();
#pragma unroll
        for (int i = 0; i < D - 2; ++i) mk[i] = mk[i + 1];
        mk[D - 2] = ops;
        __builtin_amdgcn_sched_barrier(0);
        if (pend) {                                // uniform
            store_tile(ct - 1);
            pend = false;
        }
#pragma unroll
        for (int u = 0; u < SPG; ++u) {
        const uint32_t l = SPG * kgrp + (uint32_t) u;
        if (SS * cit + l < c_nsup) {               // past the tile's last super-step: nothing
            const uint32_t slot = G % (uint32_t) D;
            const uint8_t *st = S + (SS * slot + l) * A_BYTES;
            const uint8_t *sw = S + slot * WSLOT;
            const uint32_t boff = A_REGION + (wr + li) * PB + (((4u * l + g) ^ (li & 7u)) * 16u);
            u32x4 raw[TN];
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) raw[tn] = *reinterpret_cast<const u32x4 *>(sw + boff + (uint32_t) tn * BROW16);
            i32x4v av[2][TM], bv[2][TN];
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) av[0][tm] = *reinterpret_cast<const i32x4v *>(st + aoff[0] + (uint32_t) tm * 4096u);
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
#pragma unroll
                for (int dd = 0; dd < 4; ++dd) bv[0][tn][dd] = (int32_t) ((raw[tn][dd] >> 6u) & 0x03030303u);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int f = 0; f < 4; ++f) {
                const int cu = f & 1, nx = cu ^ 1;
                if (f < 3) {
#pragma unroll
                    for (int tm = 0; tm < TM; ++tm)
                        av[nx][tm] = *reinterpret_cast<const i32x4v *>(st + aoff[f + 1] + (uint32_t) tm * 4096u);
#pragma unroll
                    for (int tn = 0; tn < TN; ++tn) {
#pragma unroll
                        for (int dd = 0; dd < 4; ++dd)
                            bv[nx][tn][dd] = (int32_t) ((raw[tn][dd] >> (4u - 2u * (uint32_t) f)) & 0x03030303u);
                    }
                }
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) {
#pragma unroll
                    for (int tm = 0; tm < TM; ++tm)
                        c[tm][tn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[cu][tm], bv[cu][tn], c[tm][tn], 0, 0, 0);
                }
                if (f < 3) {
                    constexpr int VPM = (8 * TN + TM * TN - 1) / (TM * TN);
#pragma unroll
                    for (int i = 0; i < TM * TN; ++i) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        if (i < TM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        }
        if (++cit == c_iters) {                    // tile ct done: its sums into E set ct % 2
            uint32_t *mine = reinterpret_cast<uint32_t *>(S + OFF_E + (ct & 1u) * E_SET + kgrp * E_TILE);
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) {
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr)
                        mine[(16u * (uint32_t) tm + 4u * g + (uint32_t) rr) * EP + wr + 16u * (uint32_t) tn + li] =
                            (uint32_t) c[tm][tn][rr];
                    c[tm][tn] = (i32x4v) { 0, 0, 0, 0 };
                }
            pend = true;
            cit = 0;
            if (++ct < nt) {
                c_nsup = __builtin_amdgcn_readfirstlane(R[ct].k) / 256u;
                c_iters = (c_nsup + SS - 1) / SS;
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __syncthreads();
    if (pend) store_tile(ct - 1);
    wait_vmem<0>();                                // no copy may land after the workgroup leaves
}

} // namespace

// ---------------------------------------------------------------------------
// entry points (argument lists mirrored in gfx950_shim.c)
// ---------------------------------------------------------------------------

// One workgroup per activation row: x[m][n] -> q[m][n], act[m].
extern "C" __global__ void __launch_bounds__(QUANT_THREADS)
sllm_k_quant_act(const float *__restrict__ x, uint32_t n, int8_t *__restrict__ q,
                 act_t *__restrict__ act) {
    __shared__ float red_f[QUANT_THREADS / 64];
    __shared__ int red_i[QUANT_THREADS / 64];
    const size_t row = blockIdx.x;
    quant_row(x + row * n, n, q + row * n, act + row, red_f, red_i);
}

// One workgroup per entry of a list of rows of any widths (every distinct
// activation of a batch of GEMVs in one launch).
struct quant_job {
    const float *x;
    int8_t      *q;
    act_t       *act;
    uint32_t     n;
    uint32_t     pad;
};

extern "C" __global__ void __launch_bounds__(QUANT_THREADS)
sllm_k_quant_list(const quant_job *__restrict__ jobs) {
    __shared__ float red_f[QUANT_THREADS / 64];
    __shared__ int red_i[QUANT_THREADS / 64];
    const quant_job j = jobs[blockIdx.x];
    quant_row(j.x, j.n, j.q, j.act, red_f, red_i);
}

// The host-pointer row's quantiser (one workgroup): x lives in pinned host
// memory, so every load of it crosses PCIe. The first QH_REG * 4 *
// QH_THREADS values are loaded at once into registers and read once (the
// rest, if any, twice); q and act are written to device memory, for the
// GEMVs that follow, and to pinned host memory, for the caller; then `seq`
// is stored to the pinned word `done` with system-scope release, for the
// host to wait on. quant_row's arithmetic (max of |x| dropping NaN, s = 127 /
// amax, quant_one, integer sum), so the same bits.
constexpr int QH_THREADS = 1024, QH_REG = 4;

extern "C" __global__ void __launch_bounds__(QH_THREADS)
sllm_k_quant_host(const float *__restrict__ x, uint32_t n, int8_t *__restrict__ q_dev,
                  act_t *__restrict__ act_dev, int8_t *__restrict__ q_host, act_t *__restrict__ act_host,
                  uint32_t *done, uint32_t seq) {
    __shared__ float red_f[QH_THREADS / 64];
    __shared__ int red_i[QH_THREADS / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool vec = (n & 3u) == 0;
    constexpr uint32_t STEP = 4u * QH_THREADS;
    f32x4 v[QH_REG];
    float m = 0.0f;
    if (vec) {
#pragma unroll
        for (int r = 0; r < QH_REG; ++r) {
            const uint32_t i = 4u * tid + (uint32_t) r * STEP;
            v[r] = i < n ? *G_CAST(const f32x4, x + i) : f32x4 { 0.0f, 0.0f, 0.0f, 0.0f };
        }
#pragma unroll
        for (int r = 0; r < QH_REG; ++r)
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v[r][0]), fabsf(v[r][1])), fmaxf(fabsf(v[r][2]), fabsf(v[r][3]))));
        for (uint32_t i = 4u * tid + QH_REG * STEP; i < n; i += STEP) {
            const f32x4 t = *G_CAST(const f32x4, x + i);
            m = fmaxf(m, fmaxf(fmaxf(fabsf(t[0]), fabsf(t[1])), fmaxf(fabsf(t[2]), fabsf(t[3]))));
        }
    } else {
        for (uint32_t i = tid; i < n; i += QH_THREADS) m = fmaxf(m, fabsf(G_CAST(const float, x)[i]));
    }
    m = wave_max(m);
    if (lane == 0) red_f[wave] = m;
    __syncthreads();
    m = red_f[0];
#pragma unroll
    for (int w = 1; w < QH_THREADS / 64; ++w) m = fmaxf(m, red_f[w]);
    const float s = m > 0.0f ? 127.0f / m : 0.0f;

    int sum = 0;
    auto put4 = [&](uint32_t i, const f32x4 t) {
        const int a = quant_one(t[0] * s), b = quant_one(t[1] * s);
        const int c = quant_one(t[2] * s), d = quant_one(t[3] * s);
        sum += a + b + c + d;
        const uint32_t packed = (uint32_t) (a & 0xff) | ((uint32_t) (b & 0xff) << 8) |
                                ((uint32_t) (c & 0xff) << 16) | ((uint32_t) (d & 0xff) << 24);
        *G_CAST(uint32_t, q_dev + i) = packed;
        *G_CAST(uint32_t, q_host + i) = packed;
    };
    if (vec) {
#pragma unroll
        for (int r = 0; r < QH_REG; ++r) {
            const uint32_t i = 4u * tid + (uint32_t) r * STEP;
            if (i < n) put4(i, v[r]);
        }
        for (uint32_t i = 4u * tid + QH_REG * STEP; i < n; i += STEP) put4(i, *G_CAST(const f32x4, x + i));
    } else {
        for (uint32_t i = tid; i < n; i += QH_THREADS) {
            const int a = quant_one(G_CAST(const float, x)[i] * s);
            sum += a;
            G_CAST(int8_t, q_dev)[i] = (int8_t) a;
            G_CAST(int8_t, q_host)[i] = (int8_t) a;
        }
    }
    sum = wave_sum(sum);
    if (lane == 0) red_i[wave] = sum;
    // every wave makes its q stores visible to the host itself (a
    // system-scope release of its own), before the barrier after which
    // thread 0 publishes `done`: the host reads q as soon as it sees it
    __threadfence_system();
    __syncthreads();
    if (tid == 0) {
        int t = 0;
#pragma unroll
        for (int w = 0; w < QH_THREADS / 64; ++w) t += red_i[w];
        G_CAST(float, act_dev)[0] = s;
        G_CAST(int32_t, act_dev)[1] = t;
        G_CAST(float, act_host)[0] = s;
        G_CAST(int32_t, act_host)[1] = t;
        __hip_atomic_store(done, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// Completion word for the host-pointer row: launched behind a kernel on the
// same stream, so it runs once that kernel has finished and released its
// writes; the host waits on `done` instead of a stream synchronisation.
extern "C" __global__ void __launch_bounds__(64)
sllm_k_host_done(uint32_t *done, uint32_t seq) {
    if (threadIdx.x == 0) __hip_atomic_store(done, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Slab GEMV: blocks of SLAB_THREADS, static LDS. With descs null this is a
// single-job launch: slab blockIdx.x of gridDim.x slabs of `single`.
extern "C" __global__ void __launch_bounds__(SLAB_THREADS)
sllm_k_gemv_slab(const gemv_job *__restrict__ jobs, const wg_desc *__restrict__ descs,
                 uint32_t n_wg, gemv_job single, uint32_t single_flags) {
    __shared__ slab_shared S;
    gemv_job job;
    uint32_t slab, n_slabs, flags;
    if (descs != nullptr) {
        const wg_desc d = descs[xcd_slot(n_wg)];
        if (d.b == 0) return;
        job = jobs[d.job];
        slab = d.a;
        n_slabs = d.b;
        flags = d.flags;
    } else {
        job = single;
        slab = blockIdx.x;
        n_slabs = gridDim.x;
        flags = (single_flags & ~WG_PUBLISH) | (blockIdx.x == 0 ? WG_PUBLISH : 0u);
    }
    const bool quant = job.x != nullptr;
    if (job.variant == 0) {                                                      // K <= 2560
        if (quant) slab_block<8, 5, 3, 1, true>(job, slab, n_slabs, flags, S);
        else slab_block<8, 5, 3, 1, false>(job, slab, n_slabs, flags, S);
    } else {                                                                     // K <= 7168
        if (quant) slab_block<16, 7, 7, 2, true>(job, slab, n_slabs, flags, S);
        else slab_block<16, 7, 7, 2, false>(job, slab, n_slabs, flags, S);
    }
}

// Streaming GEMV: any block size up to 1024, K bytes of dynamic LDS.
#define SLLM_STREAM_ENTRY(L)                                                                  \
    extern "C" __global__ void __launch_bounds__(1024)                                        \
    sllm_k_gemv_stream_l##L(const gemv_job *__restrict__ jobs, const wg_desc *__restrict__ descs, \
                            uint32_t n_wg, gemv_job single, uint32_t single_rows) {           \
        gemv_job job;                                                                         \
        uint32_t row_begin, row_end;                                                          \
        if (!stream_share(jobs, descs, n_wg, single, single_rows, job, row_begin, row_end)) return; \
        stream_block<L>(job, row_begin, row_end);                                             \
    }

SLLM_STREAM_ENTRY(4)
SLLM_STREAM_ENTRY(8)
SLLM_STREAM_ENTRY(16)


// Batched ternary GEMM, blocks of 256: grid (row tiles, token tiles). One
// instantiation per tile shape the host picks by token count:
//   _s1x1  16 tokens x 16 rows, K split over the four waves
//   _2x2   32 tokens x 128 rows      _4x2   64 tokens x 128 rows
//   _l128  128 tokens x 128 rows staged through LDS (K % 256 == 0)
//   _dl<TM>x<TN>  16 TM tokens x 64 TN rows, direct-load ring (K % 256 == 0)
extern "C" __global__ void __launch_bounds__(256)
sllm_k_gemm_mfma_s1x1(gemm_args G) { gemm_block<1, 1, 4>(G); }
extern "C" __global__ void __launch_bounds__(256)
sllm_k_gemm_mfma_2x2(gemm_args G) { gemm_block<2, 2, 1>(G); }
extern "C" __global__ void __launch_bounds__(256)
sllm_k_gemm_mfma_4x2(gemm_args G) { gemm_block<4, 2, 1>(G); }
extern "C" __global__ void __launch_bounds__(256)
sllm_k_gemm_mfma_l128(gemm_args G) { gemm_lds_block<false>(G); }
extern "C" __global__ void __launch_bounds__(256)
sllm_k_gemm_mfma_l128s(gemm_args G) { gemm_lds_block<true>(G); }
extern "C" __global__ void __launch_bounds__(256)
sllm_k_gemm_dl1x1(gemm_args G) { gemm_dl_block<1, 1, 4>(G); }
extern "C" __global__ void __launch_bounds__(256)
sllm_k_gemm_dl2x1(gemm_args G) { gemm_dl_block<2, 1, 4>(G); }
extern "C" __global__ void __launch_bounds__(256)
sllm_k_gemm_dl2x2(gemm_args G) { gemm_dl_block<2, 2, 4>(G); }
extern "C" __global__ void __launch_bounds__(256)
sllm_k_gemm_dl4x4(gemm_args G) { gemm_dl_block<4, 4, 2>(G); }
extern "C" __global__ void __launch_bounds__(512)
sllm_k_gemm_dk4x4(gemm_args G) { gemm_dl_block<4, 4, 4, 2>(G); }
extern "C" __global__ void __launch_bounds__(512)
sllm_k_gemm_dk4x2(gemm_args G) { gemm_dl_block<4, 2, 4, 2>(G); }
extern "C" __global__ void __launch_bounds__(512)
sllm_k_gemm_dk2x4(gemm_args G) { gemm_dl_block<2, 4, 4, 2>(G); }
extern "C" __global__ void __launch_bounds__(512)
sllm_k_gemm_dk2x2(gemm_args G) { gemm_dl_block<2, 2, 4, 2>(G); }
// a chunk's Q + K + V with the cache store in the epilogue (gemm_rope)
extern "C" __global__ void __launch_bounds__(512)
sllm_k_gemm_dk2x2_rope(gemm_args G, gemm_rope R) { gemm_dl_block<2, 2, 4, 2, true>(G, &R); }
extern "C" __global__ void __launch_bounds__(512)
sllm_k_gemm_dk4x4_rope(gemm_args G, gemm_rope R) { gemm_dl_block<4, 4, 4, 2, true>(G, &R); }
// gate + up with silu(gate) * up in the epilogue (gemm_dl_glu)
extern "C" __global__ void __launch_bounds__(512)
sllm_k_gemm_dk2x2_glu(gemm_args G) { gemm_dl_glu<2, 2, 4>(G); }
extern "C" __global__ void __launch_bounds__(512)
sllm_k_gemm_dk4x4_glu(gemm_args G) { gemm_dl_glu<4, 4, 4>(G); }
// one tensor with a residual added in the epilogue (gemm_dl_res), in the
// shapes of dk2x2, dk4x4, dq1x1 and dq2x1
extern "C" __global__ void __launch_bounds__(512)
sllm_k_gemm_dk2x2_res(gemm_args G, const float *res) { gemm_dl_res<2, 2, 4, 2>(G, res); }
extern "C" __global__ void __launch_bounds__(512)
sllm_k_gemm_dk4x4_res(gemm_args G, const float *res) { gemm_dl_res<4, 4, 4, 2>(G, res); }
extern "C" __global__ void __launch_bounds__(1024)
sllm_k_gemm_dq1x1_res(gemm_args G, const float *res) { gemm_dl_res<1, 1, 16, 4>(G, res); }
extern "C" __global__ void __launch_bounds__(1024)
sllm_k_gemm_dq2x1_res(gemm_args G, const float *res) { gemm_dl_res<2, 1, 12, 4>(G, res); }
// sixteen waves in four K groups over a 16 x 64 / 32 x 64 tile: for grids
// of fewer workgroups than CUs (a lone tensor against a few tokens), each
// group walks a quarter of the super-steps
extern "C" __global__ void __launch_bounds__(1024)
sllm_k_gemm_dq1x1(gemm_args G) { gemm_dl_block<1, 1, 16, 4>(G); }
extern "C" __global__ void __launch_bounds__(1024)
sllm_k_gemm_dq2x1(gemm_args G) { gemm_dl_block<2, 1, 12, 4>(G); }

// the same tiles over a plan's table of tensors
extern "C" __global__ void __launch_bounds__(256)
sllm_k_gemm_tdl1x1(gemm_table T) { gemm_dl_table<1, 1, 4>(T); }
extern "C" __global__ void __launch_bounds__(256)
sllm_k_gemm_tdl2x1(gemm_table T) { gemm_dl_table<2, 1, 4>(T); }
extern "C" __global__ void __launch_bounds__(512)
sllm_k_gemm_tdk2x2(gemm_table T) { gemm_dl_table<2, 2, 4, 2>(T); }
extern "C" __global__ void __launch_bounds__(512)
sllm_k_gemm_tdk4x2(gemm_table T) { gemm_dl_table<4, 2, 4, 2>(T); }
extern "C" __global__ void __launch_bounds__(512)
sllm_k_gemm_tdk4x4(gemm_table T) { gemm_dl_table<4, 4, 4, 2>(T); }

// a plan of a few tokens as one stream per workgroup (16 x 128 tiles)
extern "C" __global__ void __launch_bounds__(GS_THREADS)
sllm_k_gemm_s1(gemm_stream P) { gemm_stream_body<4>(P); }

// ---------------------------------------------------------------------------
// calibration kernels: a plain copy and a read-only checksum of known size,
// used to scale HBM counters and to measure the achievable bandwidth beside
// the GEMV. n16 counts 16-byte words.
// ---------------------------------------------------------------------------

extern "C" __global__ void __launch_bounds__(256)
sllm_k_copy(const u32x4 *__restrict__ src, u32x4 *__restrict__ dst, uint64_t n16) {
    const uint64_t stride = (uint64_t) gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
    }
}

// XOR of every 32-bit word, one partial per workgroup (out[blockIdx.x]).
extern "C" __global__ void __launch_bounds__(256)
sllm_k_checksum(const u32x4 *__restrict__ src, uint64_t n16, uint32_t *__restrict__ out) {
    __shared__ uint32_t red[4];
    const uint64_t stride = (uint64_t) gridDim.x * blockDim.x;
    u32x4 acc = { 0, 0, 0, 0 };
    for (uint64_t i = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        acc ^= __builtin_nontemporal_load(src + i);
    }
    uint32_t v = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v ^= (uint32_t) __shfl_xor((int) v, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}
