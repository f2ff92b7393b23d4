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

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Global-address-space views. Pointers read out of a job table in memory are
// generic to the compiler, which would then emit flat loads: those count
// against both memory counters, so every wait becomes a full drain and the
// weight prefetch stops overlapping. Casting to address space 1 keeps them
// global loads/stores. Only native vector and scalar types go through these
// casts: copying a HIP struct type (float4, uint4) passes a generic reference
// to its copy constructor and turns the access back into a flat one.
#define GLOBAL __attribute__((address_space(1)))
#define G_CAST(T, p) ((GLOBAL T *) (p))

struct act_t {          // layout of sllm_i2s_act (include/saphira_llm/i2s_gemm.h:37-40)
    float   scale;      // 127 / amax, 0 for an all-zero row
    int32_t sum;        // sum of the quantised values
};

// ---------------------------------------------------------------------------
// wave / block reductions
// ---------------------------------------------------------------------------

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Sum over aligned groups of LPR lanes with DPP moves. Every lane of the wave
// must be active: callers keep the reduction out of divergent code.
template <int LPR>
__device__ __forceinline__ int group_sum(int v) {
    static_assert(LPR == 4 || LPR == 8 || LPR == 16, "lanes per row");
    v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);    // quad_perm [1,0,3,2]
    v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);    // quad_perm [2,3,0,1]
    if (LPR >= 8) v += __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false);  // row_half_mirror
    if (LPR >= 16) v += __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, false); // row_mirror
    return v;
}

// ---------------------------------------------------------------------------
// activation quantiser (src/i2s_gemm.c:45-83)
// ---------------------------------------------------------------------------

// (int) roundf(v) as the reference's x86-64 build evaluates it: cvttss2si
// yields INT32_MIN for NaN and for |v| >= 2^31, which the clamp then maps to
// -128. (Reached only when amax is so small that 127/amax overflows.)
__device__ __forceinline__ int quant_one(float xs) {
    const float r = roundf(xs);
    int v = fabsf(r) < 2147483648.0f ? (int) r : INT32_MIN;
    v = v > 127 ? 127 : v;
    v = v < -128 ? -128 : v;
    return v;
}

constexpr int QUANT_THREADS = 256;

__device__ __forceinline__ void quant_row(const float *__restrict__ x, uint32_t n,
                                          int8_t *__restrict__ q, act_t *__restrict__ act,
                                          float *red_f, int *red_i) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool vec = (n & 3u) == 0;

    // pass 1: amax = max |x|. fmaxf drops NaN exactly as `a > amax` does.
    float m = 0.0f;
    if (vec) {
        for (uint32_t i = 4u * tid; i < n; i += 4u * QUANT_THREADS) {
            const f32x4 v = *G_CAST(const f32x4, x + i);
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
        }
    } else {
        for (uint32_t i = tid; i < n; i += QUANT_THREADS) m = fmaxf(m, fabsf(G_CAST(const float, x)[i]));
    }
    m = wave_max(m);
    if (lane == 0) red_f[wave] = m;
    __syncthreads();
    m = red_f[0];
#pragma unroll
    for (int w = 1; w < QUANT_THREADS / 64; ++w) m = fmaxf(m, red_f[w]);

    // reciprocal scale with IEEE division, 0 for an all-zero row
    const float s = m > 0.0f ? 127.0f / m : 0.0f;

    // pass 2: q = clamp(round-half-away(x*s)), running sum
    int sum = 0;
    if (vec) {
        for (uint32_t i = 4u * tid; i < n; i += 4u * QUANT_THREADS) {
            const f32x4 v = *G_CAST(const f32x4, x + i);
            const int a = quant_one(v[0] * s), b = quant_one(v[1] * s);
            const int c = quant_one(v[2] * s), d = quant_one(v[3] * s);
            sum += a + b + c + d;
            *G_CAST(uint32_t, q + i) =
                (uint32_t) (a & 0xff) | ((uint32_t) (b & 0xff) << 8) |
                ((uint32_t) (c & 0xff) << 16) | ((uint32_t) (d & 0xff) << 24);
        }
    } else {
        for (uint32_t i = tid; i < n; i += QUANT_THREADS) {
            const int a = quant_one(G_CAST(const float, x)[i] * s);
            sum += a;
            G_CAST(int8_t, q)[i] = (int8_t) a;
        }
    }
    sum = wave_sum(sum);
    if (lane == 0) red_i[wave] = sum;
    __syncthreads();
    if (tid == 0) {
        int t = 0;
#pragma unroll
        for (int w = 0; w < QUANT_THREADS / 64; ++w) t += red_i[w];
        G_CAST(float, act)[0] = s;
        G_CAST(int32_t, act)[1] = t;
    }
}

// ---------------------------------------------------------------------------
// ternary dot over one 16-byte chunk of a packed row
// ---------------------------------------------------------------------------
//
// A 16-byte chunk c of a row is half h = c & 1 of block b = c >> 1: bytes
// (lanes) 16h..16h+15 of the block. Dword d of the chunk holds lanes
// 16h+4d..16h+4d+3, and field f of byte j of that dword is element
// 128b + 32f + 16h + 4d + j, so it pairs with byte j of the activation dword
// at q[128b + 32f + 16h + 4d]: a plain 4-way int8 dot per (dword, field).
//
// The codes are isolated in place instead of shifted down: masking field 3,
// 2, 1 leaves code*1, code*4, code*16 in each byte, and field 0 shifted right
// by one leaves code*32. All stay below 128, so they are valid signed int8
// operands of sdot4; each field keeps its own int32 accumulator and the
// scale factors are divided out exactly once at the end.

struct dot4acc {
    int f0, f1, f2, f3;
};

__device__ __forceinline__ void chunk_dot(const u32x4 wv, const int8_t *__restrict__ a,
                                          dot4acc &acc) {
    const i32x4 q0 = *reinterpret_cast<const i32x4 *>(a);        // field 0: q[.. + 0 ..]
    const i32x4 q1 = *reinterpret_cast<const i32x4 *>(a + 32);   // field 1
    const i32x4 q2 = *reinterpret_cast<const i32x4 *>(a + 64);   // field 2
    const i32x4 q3 = *reinterpret_cast<const i32x4 *>(a + 96);   // field 3
    const u32x4 wd = wv;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        acc.f3 = __builtin_amdgcn_sdot4((int) (wd[d] & 0x03030303u), q3[d], acc.f3, false);
        acc.f2 = __builtin_amdgcn_sdot4((int) (wd[d] & 0x0C0C0C0Cu), q2[d], acc.f2, false);
        acc.f1 = __builtin_amdgcn_sdot4((int) (wd[d] & 0x30303030u), q1[d], acc.f1, false);
        acc.f0 = __builtin_amdgcn_sdot4((int) ((wd[d] >> 1) & 0x60606060u), q0[d], acc.f0, false);
    }
}

__device__ __forceinline__ int finish(const dot4acc &acc) {
    // each accumulator is an exact multiple of its field weight
    return acc.f3 + (acc.f2 >> 2) + (acc.f1 >> 4) + (acc.f0 >> 5);
}

// ---------------------------------------------------------------------------
// GEMV jobs
// ---------------------------------------------------------------------------

struct gemv_job {
    const uint8_t *w;          // packed tensor (codes + 32-byte tail)
    const float   *x;          // f32 activation quantised in-kernel, or null
    int8_t        *q;          // int8 activation: read when x is null, else optional output
    act_t         *act;        // its scale/sum: read when x is null, else optional output
    float         *out_f;      // epilogue output, or null
    int32_t       *out_i;      // raw int32 dots, or null
    uint32_t       n_rows;     // N
    uint32_t       k;          // K, a multiple of 128
    uint32_t       wg_begin;   // first workgroup of this job (group launches)
    uint32_t       rows_per_wg;
    uint32_t       variant;    // row-group geometry (row-group kernel only)
    uint32_t       pad;
};

// w_scale / act_scale, the epilogue's once-per-column factor (i2s_gemm.c:288)
__device__ __forceinline__ float epilogue_post(const gemv_job &job, float act_scale) {
    const float ws = *G_CAST(const float, job.w + (size_t) job.n_rows * (job.k >> 2));
    return ws / act_scale;
}

__device__ __forceinline__ void store_row(const gemv_job &job, uint32_t row, int dot, int32_t asum,
                                          float post) {
    if (job.out_i != nullptr) G_CAST(int32_t, job.out_i)[row] = dot;
    if (job.out_f != nullptr) G_CAST(float, job.out_f)[row] = (float) (dot - asum) * post;
}

// Copy the K-byte activation into LDS (the caller synchronises).
__device__ __forceinline__ void stage_q(const int8_t *__restrict__ q, uint32_t k, int8_t *q_lds) {
    for (uint32_t i = 16u * threadIdx.x; i < k; i += 16u * blockDim.x) {
        *reinterpret_cast<u32x4 *>(q_lds + i) = *G_CAST(const u32x4, q + i);
    }
}

constexpr int MAX_WAVES = 16;

// The activation of a job, in LDS, with its scale and sum. Either staged from
// a quantised row, or quantised here from x -- the same operations as
// quant_row, so every workgroup of the job derives identical bits. All
// threads of the block call this; it ends with q_lds complete and visible.
__device__ __forceinline__ void activation_to_lds(const gemv_job &job, uint32_t local_wg,
                                                  int8_t *q_lds, float *red_f, int *red_i,
                                                  float &scale, int32_t &sum) {
    const int tid = threadIdx.x, nthr = blockDim.x, lane = tid & 63, wave = tid >> 6;
    const int nw = nthr >> 6;
    const uint32_t k = job.k;
    if (job.x == nullptr) {
        stage_q(job.q, k, q_lds);
        // act is only required (and only given) when the epilogue runs
        scale = 0.0f;
        sum = 0;
        if (job.act != nullptr) {
            scale = G_CAST(const float, job.act)[0];
            sum = G_CAST(const int32_t, job.act)[1];
        }
        __syncthreads();
        return;
    }
    const float *x = job.x;
    float m = 0.0f;
    for (uint32_t i = 4u * tid; i < k; i += 4u * nthr) {
        const f32x4 v = *G_CAST(const f32x4, x + i);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    }
    m = wave_max(m);
    if (lane == 0) red_f[wave] = m;
    __syncthreads();
    m = red_f[0];
    for (int w = 1; w < nw; ++w) m = fmaxf(m, red_f[w]);
    const float s = m > 0.0f ? 127.0f / m : 0.0f;
    int ls = 0;
    for (uint32_t i = 4u * tid; i < k; i += 4u * nthr) {
        const f32x4 v = *G_CAST(const f32x4, x + i);
        const int a = quant_one(v[0] * s), b = quant_one(v[1] * s);
        const int c = quant_one(v[2] * s), d = quant_one(v[3] * s);
        ls += a + b + c + d;
        *reinterpret_cast<uint32_t *>(q_lds + i) =
            (uint32_t) (a & 0xff) | ((uint32_t) (b & 0xff) << 8) |
            ((uint32_t) (c & 0xff) << 16) | ((uint32_t) (d & 0xff) << 24);
    }
    ls = wave_sum(ls);
    if (lane == 0) red_i[wave] = ls;
    __syncthreads();
    int t = 0;
    for (int w = 0; w < nw; ++w) t += red_i[w];
    scale = s;
    sum = t;
    if (local_wg == 0) {       // one workgroup publishes the quantised row
        if (job.q != nullptr) {
            for (uint32_t i = 16u * tid; i < k; i += 16u * nthr) {
                *G_CAST(u32x4, job.q + i) = *reinterpret_cast<const u32x4 *>(q_lds + i);
            }
        }
        if (job.act != nullptr && tid == 0) {
            G_CAST(float, job.act)[0] = s;
            G_CAST(int32_t, job.act)[1] = t;
        }
    }
}

// ---------------------------------------------------------------------------
// streaming GEMV (any K up to the LDS limit): waves loop over row groups,
// 8 loads in flight per lane. Reads a quantised activation (x must be null).
// ---------------------------------------------------------------------------

constexpr int UNROLL = 8;

template <int LPR>
__device__ __forceinline__ void stream_rows(const gemv_job &job, uint32_t row_begin,
                                            uint32_t row_end, const int8_t *q_lds,
                                            int32_t asum, float post) {
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
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
        if (valid && sub == 0) store_row(job, row, dot, asum, post);
    }
}

template <int LPR>
__device__ __forceinline__ void stream_block(const gemv_job &job, uint32_t local_wg) {
    extern __shared__ __attribute__((aligned(16))) int8_t q_lds[];
    const uint32_t row_begin = local_wg * job.rows_per_wg;
    if (row_begin >= job.n_rows) return;           // uniform across the block
    const uint32_t row_end = min(job.n_rows, row_begin + job.rows_per_wg);
    stage_q(job.q, job.k, q_lds);
    __syncthreads();
    float post = 0.0f;
    int32_t asum = 0;
    if (job.out_f != nullptr) {
        post = epilogue_post(job, G_CAST(const float, job.act)[0]);
        asum = G_CAST(const int32_t, job.act)[1];
    }
    stream_rows<LPR>(job, row_begin, row_end, q_lds, asum, post);
}

// ---------------------------------------------------------------------------
// row-group GEMV. A block owns rows_per_wg consecutive rows of one job; its
// waves take turns over row groups of 64/LPR rows (LPR lanes per row, each
// lane CPL 16-byte chunks of its row), double-buffered: the loads of a
// wave's next row group are issued before the current one is reduced, so a
// wave never waits a full memory round trip between groups. The first
// group's loads are issued before the activation is built in LDS --
// quantised from x in-kernel when the job carries it -- which costs one read
// of x per block, a few percent of the block's weight bytes.
// Geometry per K class (the `variant` of a job):
//   0: LPR 8,  CPL 5    K <= 2560
//   1: LPR 16, CPL 7    K <= 7168
//   2: LPR 8,  CPL 14   K <= 7168
//   3: LPR 16, CPL 16   K <= 16384
// ---------------------------------------------------------------------------

// The loads are unconditional, so the loop stays straight-line and the
// compiler can wait for one buffer while the other is still in flight. A
// lane whose row lies past row_end, or whose chunk slot lies past the row,
// re-reads the last valid row / chunk (lines already being fetched: no extra
// HBM traffic) and rg_reduce zeroes those weights. base < row_end always.
template <int LPR, int CPL>
__device__ __forceinline__ void rg_load(const gemv_job &job, uint32_t base, uint32_t row_end,
                                        u32x4 (&buf)[CPL]) {
    const int lane = threadIdx.x & 63, sub = lane % LPR;
    const uint32_t chunks = job.k >> 6, row_bytes = job.k >> 2;
    const uint32_t row = min(base + (uint32_t) (lane / LPR), row_end - 1);
    const GLOBAL u32x4 *wr = G_CAST(const u32x4, job.w + (size_t) row * row_bytes);
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
        const uint32_t c = min((uint32_t) (sub + u * LPR), chunks - 1);
        buf[u] = __builtin_nontemporal_load(wr + c);
    }
}

template <int LPR, int CPL>
__device__ __forceinline__ void rg_reduce(const gemv_job &job, uint32_t base, uint32_t row_end,
                                          const u32x4 (&buf)[CPL], const int8_t *q_lds,
                                          int32_t asum, float post) {
    const int lane = threadIdx.x & 63, sub = lane % LPR;
    const uint32_t chunks = job.k >> 6;
    const uint32_t row = base + (uint32_t) (lane / LPR);
    const bool valid = row < row_end;
    // The activation reads are the same for every row group of the wave; left
    // alone the compiler keeps all of them in registers across the loop,
    // which halves occupancy. Re-reading them from LDS is cheaper: hide the
    // base from loop-invariant code motion.
    uint32_t lds_base = 0;
    asm volatile("" : "+v"(lds_base));
    dot4acc acc = { 0, 0, 0, 0 };
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
        const uint32_t slot = (uint32_t) (sub + u * LPR);
        const uint32_t c = min(slot, chunks - 1);
        const bool use = valid && slot < chunks;
        const u32x4 zero = { 0, 0, 0, 0 };
        chunk_dot(use ? buf[u] : zero, q_lds + lds_base + (c >> 1) * 128u + (c & 1u) * 16u, acc);
    }
    const int dot = group_sum<LPR>(finish(acc));      // whole wave active here
    if (valid && sub == 0) store_row(job, row, dot, asum, post);
}

template <int LPR, int CPL>
__device__ __forceinline__ void rowgroup_block(const gemv_job &job, uint32_t local_wg, int8_t *q_lds,
                                               float *red_f, int *red_i) {
    constexpr uint32_t RPW = 64 / LPR;
    const uint32_t wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const uint32_t row_begin = local_wg * job.rows_per_wg;
    if (row_begin >= job.n_rows) return;           // uniform across the block
    const uint32_t row_end = min(job.n_rows, row_begin + job.rows_per_wg);
    const uint32_t stride = waves * RPW;

    // wave-uniform first row of this wave's current group; a wave whose first
    // group is already past the block's rows still takes part in the barriers
    uint32_t base = row_begin + wave * RPW;
    u32x4 bufa[CPL], bufb[CPL];
    rg_load<LPR, CPL>(job, min(base, row_end - 1), row_end, bufa);

    float scale;
    int32_t asum;
    activation_to_lds(job, local_wg, q_lds, red_f, red_i, scale, asum);
    const float post = job.out_f != nullptr ? epilogue_post(job, scale) : 0.0f;

    while (base < row_end) {
        rg_load<LPR, CPL>(job, min(base + stride, row_end - 1), row_end, bufb);
        rg_reduce<LPR, CPL>(job, base, row_end, bufa, q_lds, asum, post);
        base += stride;
        if (base >= row_end) break;
        rg_load<LPR, CPL>(job, min(base + stride, row_end - 1), row_end, bufa);
        rg_reduce<LPR, CPL>(job, base, row_end, bufb, q_lds, asum, post);
        base += stride;
    }
}

// Variants are compiled into three kernel classes so that the register
// budget of the wide ones does not lower the occupancy of the common ones:
// class 0 = variants 0 and 1 (the K classes of the BitNet-2B projections),
// class 1 = variant 2, class 2 = variant 3.
template <int CLASS>
__device__ __forceinline__ void rowgroup_dispatch(const gemv_job &job, uint32_t local_wg) {
    extern __shared__ __attribute__((aligned(16))) int8_t q_lds[];
    __shared__ float red_f[MAX_WAVES];
    __shared__ int red_i[MAX_WAVES];
    if (CLASS == 0) {
        if (job.variant == 0) rowgroup_block<8, 5>(job, local_wg, q_lds, red_f, red_i);
        else rowgroup_block<16, 7>(job, local_wg, q_lds, red_f, red_i);
    } else if (CLASS == 1) {
        rowgroup_block<8, 14>(job, local_wg, q_lds, red_f, red_i);
    } else {
        rowgroup_block<16, 16>(job, local_wg, q_lds, red_f, red_i);
    }
}

// jobs are sorted by wg_begin; the block's job is the last with wg_begin <= blockIdx.x
__device__ __forceinline__ gemv_job find_job(const gemv_job *__restrict__ jobs, uint32_t n_jobs) {
    uint32_t lo = 0, hi = n_jobs;
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (jobs[mid].wg_begin <= blockIdx.x) lo = mid; else hi = mid;
    }
    return jobs[lo];
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

#define SLLM_STREAM_ENTRY(L)                                                            \
    extern "C" __global__ void __launch_bounds__(1024)                                  \
    sllm_k_gemv_l##L(gemv_job job) { stream_block<L>(job, blockIdx.x); }                \
    extern "C" __global__ void __launch_bounds__(1024)                                  \
    sllm_k_gemv_group_l##L(const gemv_job *__restrict__ jobs, uint32_t n_jobs) {        \
        const gemv_job job = find_job(jobs, n_jobs);                                    \
        stream_block<L>(job, blockIdx.x - job.wg_begin);                                \
    }

SLLM_STREAM_ENTRY(4)
SLLM_STREAM_ENTRY(8)
SLLM_STREAM_ENTRY(16)

// Row-group kernels, one per class: at most 4 waves per block.
#define SLLM_RG_ENTRY(C)                                                                \
    extern "C" __global__ void __launch_bounds__(256)                                   \
    sllm_k_gemv_rg_c##C(gemv_job job) { rowgroup_dispatch<C>(job, blockIdx.x); }        \
    extern "C" __global__ void __launch_bounds__(256)                                   \
    sllm_k_gemv_rg_group_c##C(const gemv_job *__restrict__ jobs, uint32_t n_jobs) {     \
        const gemv_job job = find_job(jobs, n_jobs);                                    \
        rowgroup_dispatch<C>(job, blockIdx.x - job.wg_begin);                           \
    }

SLLM_RG_ENTRY(0)
SLLM_RG_ENTRY(1)
SLLM_RG_ENTRY(2)

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
