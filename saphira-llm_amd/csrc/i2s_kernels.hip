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
// GEMV jobs and workgroup descriptors
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
    uint32_t       variant;    // slab kernel geometry: 0 = (8 lanes, 5 chunks), 1 = (16, 7)
    uint32_t       pad;
};

// One workgroup's share of a batch, in job `job`:
//   slab kernel      slab a of b slabs of the job (b == 0: padding); flags
//                    WG_PUBLISH
//   streaming kernel rows [a, b) (a >= b: padding)
// Empty descriptors pad the table to a multiple of 8 workgroups.
struct wg_desc {
    uint32_t job;
    uint32_t a;
    uint32_t b;
    uint32_t flags;
};

constexpr uint32_t WG_PUBLISH = 1;      // this workgroup writes the job's quantised row (q / act)

// Workgroups are dealt to the 8 XCDs round-robin by block index. Read the
// descriptor table so that XCD x runs the x-th eighth of it in order: the
// slabs of one job then share an XCD, and its L2 fetches the job's activation
// once instead of every XCD fetching it. n_wg is a multiple of 8.
__device__ __forceinline__ uint32_t xcd_slot(uint32_t n_wg) {
    return (blockIdx.x & 7u) * (n_wg >> 3) + (blockIdx.x >> 3);
}

// w_scale, the f32 after the packed codes (src/quant.c:102-106)
__device__ __forceinline__ float tensor_scale(const gemv_job &job) {
    return *G_CAST(const float, job.w + (size_t) job.n_rows * (job.k >> 2));
}

// ---------------------------------------------------------------------------
// slab GEMV (K <= 7168: every BitNet-2B projection). A workgroup of four
// waves owns a slab of consecutive rows of one job, sized by bytes so that
// every workgroup streams about the same amount of weights. Each wave walks
// groups of 64/LPR rows (LPR lanes per row, CPL 16-byte chunks per lane),
// double-buffered: the next group's loads are in flight while the current
// one is reduced, and the dots go to LDS, so no store sits between the loads
// and nothing forces the wave to drain its loads. In the prologue the
// activation loads are issued before the first weight group, so the wave
// waits only for the activation while the weights keep streaming; when the
// job carries f32 x the workgroup quantises it here (the operations of
// quant_row, so the same bits) and no quantiser launch is needed. Outputs
// and the epilogue are written at the end, coalesced.
// ---------------------------------------------------------------------------

constexpr int SLAB_THREADS = 256;
constexpr int SLAB_WAVES = SLAB_THREADS / 64;
constexpr uint32_t SLAB_MAX_K = 7168;
constexpr uint32_t SLAB_MAX_ROWS = 1024;

static_assert(8 * 5 * 64 <= SLAB_MAX_K && 16 * 7 * 64 <= SLAB_MAX_K, "slab geometries read inside the LDS row");

struct slab_shared {
    int8_t  q[SLAB_MAX_K];
    int32_t dots[SLAB_MAX_ROWS];
    float   red_f[SLAB_WAVES];
    int     red_i[SLAB_WAVES];
};

// Every load of the slab kernel is unconditional: a skipped load (a branch
// around it, or an exec-masked block the wave jumps over when no lane needs
// it) leaves the compiler unsure how many loads are outstanding where paths
// meet, and it then waits for all of them, draining the prefetch. Weights
// are read through a buffer resource bounded by the tensor's size (the host
// keeps slab tensors below 4 GiB): a chunk slot past the end of the last row
// reads zeros instead of faulting, so lane slot u is simply the lane's
// offset plus a constant. A lane whose row lies past the slab re-reads the
// slab's last row (lines already being fetched); slab_dot zeroes what it
// must not use -- those rows, and slots past the end of a row, which read
// the next row.

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tensor_rsrc(const gemv_job &job) {
    const uint32_t bytes = job.n_rows * (job.k >> 2) + 32u;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(job.w), (short) 0, (int) bytes,
                                             0x00020000);    // raw buffer, 32-bit data format
}

constexpr int CPOL_NT = 2;      // nontemporal: weights are read once

template <int LPR, int CPL>
__device__ __forceinline__ void slab_load(__amdgpu_buffer_rsrc_t rsrc, uint32_t row_bytes, uint32_t base,
                                          uint32_t last_row, u32x4 (&buf)[CPL]) {
    const int lane = threadIdx.x & 63;
    const uint32_t row = min(base + (uint32_t) (lane / LPR), last_row);
    const uint32_t off = row * row_bytes + (uint32_t) (lane % LPR) * 16u;
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
        buf[u] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int) (off + (uint32_t) (u * LPR * 16)), 0, CPOL_NT);
    }
}

// Dots of one wave's rows [row0, row0 + 64/LPR) (rows past n_rows masked)
// into dots[0 .. 64/LPR).
template <int LPR, int CPL>
__device__ __forceinline__ void slab_dot(uint32_t chunks, uint32_t row0, uint32_t n_rows,
                                         const u32x4 (&buf)[CPL], const int8_t *q_lds, int32_t *dots) {
    const int lane = threadIdx.x & 63, sub = lane % LPR;
    const uint32_t row = row0 + (uint32_t) (lane / LPR);
    const bool valid = row < n_rows;
    // Chunk slot u of this lane is chunk sub + u*LPR: with LPR even its
    // activation quarter starts at (sub/2)*128 + (sub&1)*16 + u*LPR*64, one
    // base plus constant offsets. Slots past the row (zeroed below) read
    // inside the LDS row all the same: LPR*CPL*64 <= SLAB_MAX_K. The base is
    // hidden from loop-invariant code motion: hoisted, the activation reads
    // of every group would stay in registers across the loop.
    uint32_t lds_lane = (uint32_t) (sub >> 1) * 128u + (uint32_t) (sub & 1) * 16u;
    asm volatile("" : "+v"(lds_lane));
    dot4acc acc = { 0, 0, 0, 0 };
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
        const bool use = valid && (uint32_t) (sub + u * LPR) < chunks;
        const u32x4 zero = { 0, 0, 0, 0 };
        chunk_dot(use ? buf[u] : zero, q_lds + lds_lane + (uint32_t) (u * LPR * 64), acc);
    }
    const int dot = group_sum<LPR>(finish(acc));      // whole wave active here
    if (valid && sub == 0) dots[lane / LPR] = dot;
}

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
    const uint32_t k = job.k, chunks = k >> 6, row_bytes = k >> 2;
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
    int32_t asum = 0;
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
    const float ws = *G_CAST(const float, ws_at);
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
        int ls = 0;
#pragma unroll
        for (int u = 0; u < XV; ++u) {
            const uint32_t i = 4u * (uint32_t) (tid + u * SLAB_THREADS);
            if (i < k) {
                const f32x4 v = xv[u];
                const int a = quant_one(v[0] * s), b = quant_one(v[1] * s);
                const int c = quant_one(v[2] * s), d = quant_one(v[3] * s);
                ls += a + b + c + d;
                *reinterpret_cast<uint32_t *>(S.q + i) =
                    (uint32_t) (a & 0xff) | ((uint32_t) (b & 0xff) << 8) |
                    ((uint32_t) (c & 0xff) << 16) | ((uint32_t) (d & 0xff) << 24);
            }
        }
        ls = wave_sum(ls);
        if (lane == 0) S.red_i[wave] = ls;
        __syncthreads();
        int t = 0;
#pragma unroll
        for (int w = 0; w < SLAB_WAVES; ++w) t += S.red_i[w];
        scale = s;
        asum = t;
    } else {
#pragma unroll
        for (int u = 0; u < QV; ++u) {
            const uint32_t i = 16u * (uint32_t) (tid + u * SLAB_THREADS);
            if (i < k) *reinterpret_cast<u32x4 *>(S.q + i) = qv[u];
        }
        __syncthreads();
    }

    // (4) the groups, double-buffered: pairs of groups with the next group
    // always loaded (the last one again past the end) before the current one
    // is reduced, then a trailing odd group. The loop has one exit and no
    // load behind a branch, so every wait names exactly the buffer it needs.
    // Dots of group t go to S.dots[t*G ..].
    int32_t *dots = S.dots + wave_row;
    uint32_t t = 0;
    for (uint32_t pair = 0; pair < T / 2; ++pair) {
        slab_load<LPR, CPL>(rsrc, row_bytes, group_row(t + 1), last_row, bufb);
        slab_dot<LPR, CPL>(chunks, group_row(t), n_rows, bufa, S.q, dots + t * G);
        ++t;
        slab_load<LPR, CPL>(rsrc, row_bytes, group_row(t + 1), last_row, bufa);
        slab_dot<LPR, CPL>(chunks, group_row(t), n_rows, bufb, S.q, dots + t * G);
        ++t;
    }
    if (T & 1u) slab_dot<LPR, CPL>(chunks, group_row(t), n_rows, bufa, S.q, dots + t * G);
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
