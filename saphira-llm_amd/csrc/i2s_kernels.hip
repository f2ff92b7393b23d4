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
            const float4 v = *reinterpret_cast<const float4 *>(x + i);
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    } else {
        for (uint32_t i = tid; i < n; i += QUANT_THREADS) m = fmaxf(m, fabsf(x[i]));
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
            const float4 v = *reinterpret_cast<const float4 *>(x + i);
            const int a = quant_one(v.x * s), b = quant_one(v.y * s);
            const int c = quant_one(v.z * s), d = quant_one(v.w * s);
            sum += a + b + c + d;
            *reinterpret_cast<uint32_t *>(q + i) =
                (uint32_t) (a & 0xff) | ((uint32_t) (b & 0xff) << 8) |
                ((uint32_t) (c & 0xff) << 16) | ((uint32_t) (d & 0xff) << 24);
        }
    } else {
        for (uint32_t i = tid; i < n; i += QUANT_THREADS) {
            const int a = quant_one(x[i] * s);
            sum += a;
            q[i] = (int8_t) a;
        }
    }
    sum = wave_sum(sum);
    if (lane == 0) red_i[wave] = sum;
    __syncthreads();
    if (tid == 0) {
        int t = 0;
#pragma unroll
        for (int w = 0; w < QUANT_THREADS / 64; ++w) t += red_i[w];
        act->scale = s;
        act->sum = t;
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
    const int4 a0 = *reinterpret_cast<const int4 *>(a);        // field 0: q[.. + 0 ..]
    const int4 a1 = *reinterpret_cast<const int4 *>(a + 32);   // field 1
    const int4 a2 = *reinterpret_cast<const int4 *>(a + 64);   // field 2
    const int4 a3 = *reinterpret_cast<const int4 *>(a + 96);   // field 3
    const uint32_t wd[4] = { wv[0], wv[1], wv[2], wv[3] };
    const int q0[4] = { a0.x, a0.y, a0.z, a0.w };
    const int q1[4] = { a1.x, a1.y, a1.z, a1.w };
    const int q2[4] = { a2.x, a2.y, a2.z, a2.w };
    const int q3[4] = { a3.x, a3.y, a3.z, a3.w };
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
// GEMV: one wave per group of 64/LPR rows, LPR lanes per row
// ---------------------------------------------------------------------------

struct gemv_job {
    const uint8_t *w;      // packed tensor (codes + 32-byte tail)
    const int8_t  *q;      // quantised activation, K bytes
    const act_t   *act;    // its scale and sum (needed for out_f)
    float         *out_f;  // epilogue output, or null
    int32_t       *out_i;  // raw int32 dots, or null
    uint32_t       n_rows; // N
    uint32_t       k;      // K, a multiple of 128
    uint32_t       wg_begin;  // first workgroup of this job (group launches)
    uint32_t       rows_per_wg;
};

constexpr int UNROLL = 8;   // 16-byte weight loads in flight per lane

template <int LPR>
__device__ __forceinline__ void gemv_rows(const gemv_job &job, uint32_t row_begin,
                                          uint32_t row_end, const int8_t *q_lds) {
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const int sub = lane % LPR;
    const uint32_t k = job.k, chunks = k >> 6, row_bytes = k >> 2;

    float post = 0.0f;
    int32_t asum = 0;
    if (job.out_f != nullptr) {
        float ws;
        __builtin_memcpy(&ws, job.w + (size_t) job.n_rows * row_bytes, sizeof ws);
        const act_t a = *job.act;
        post = ws / a.scale;          // once per activation column (i2s_gemm.c:288)
        asum = a.sum;
    }

    for (uint32_t r0 = row_begin + (uint32_t) wave * RPW; r0 < row_end; r0 += (uint32_t) waves * RPW) {
        const uint32_t row = r0 + (uint32_t) (lane / LPR);
        const bool valid = row < row_end;
        const u32x4 *wr = reinterpret_cast<const u32x4 *>(job.w + (size_t) (valid ? row : row_begin) * row_bytes);
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
            if (job.out_i != nullptr) job.out_i[row] = dot;
            if (job.out_f != nullptr) job.out_f[row] = (float) (dot - asum) * post;
        }
    }
}

__device__ __forceinline__ void stage_q(const int8_t *__restrict__ q, uint32_t k, int8_t *q_lds) {
    for (uint32_t i = 16u * threadIdx.x; i < k; i += 16u * blockDim.x) {
        *reinterpret_cast<uint4 *>(q_lds + i) = *reinterpret_cast<const uint4 *>(q + i);
    }
    __syncthreads();
}

template <int LPR>
__device__ __forceinline__ void gemv_block(const gemv_job &job, uint32_t local_wg) {
    extern __shared__ __attribute__((aligned(16))) int8_t q_lds[];
    const uint32_t row_begin = local_wg * job.rows_per_wg;
    if (row_begin >= job.n_rows) return;           // uniform across the block
    const uint32_t row_end = min(job.n_rows, row_begin + job.rows_per_wg);
    stage_q(job.q, job.k, q_lds);
    gemv_rows<LPR>(job, row_begin, row_end, q_lds);
}

template <int LPR>
__device__ __forceinline__ void gemv_group_block(const gemv_job *__restrict__ jobs, uint32_t n_jobs) {
    // jobs are sorted by wg_begin; find the last with wg_begin <= blockIdx.x
    uint32_t lo = 0, hi = n_jobs;
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (jobs[mid].wg_begin <= blockIdx.x) lo = mid; else hi = mid;
    }
    const gemv_job job = jobs[lo];
    gemv_block<LPR>(job, blockIdx.x - job.wg_begin);
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

#define SLLM_GEMV_ENTRY(L)                                                             \
    extern "C" __global__ void __launch_bounds__(1024)                                 \
    sllm_k_gemv_l##L(gemv_job job) { gemv_block<L>(job, blockIdx.x); }                 \
    extern "C" __global__ void __launch_bounds__(1024)                                 \
    sllm_k_gemv_group_l##L(const gemv_job *__restrict__ jobs, uint32_t n_jobs) {       \
        gemv_group_block<L>(jobs, n_jobs);                                             \
    }

SLLM_GEMV_ENTRY(4)
SLLM_GEMV_ENTRY(8)
SLLM_GEMV_ENTRY(16)

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
