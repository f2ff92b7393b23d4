// i2s_device.h -- device building blocks shared by the gfx950 code objects
// (i2s_kernels.hip: GEMV kernels; decode_kernels.hip: the decode step).
//
// Packed I2_S tensor, exactly as stored in the GGUF (src/quant.c:72-106,
// FORMAT.md:119-157): an N x K matrix is N rows of K/4 bytes, row r at byte
// r*K/4, followed by a 32-byte tail whose first 4 bytes are the f32 per-tensor
// scale (offset N*K/4). Within a row, 128-element block b is 32 bytes at 32*b;
// byte l of the block holds elements 128*b + 32*f + l for fields f = 0..3 at
// bit shift 6 - 2*f (field 0 in the top two bits). Codes {0,1,2} stand for
// ternary {-1,0,+1}.
#ifndef SLLM_I2S_DEVICE_H
#define SLLM_I2S_DEVICE_H

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

// ggml_v_expf, one lane (src/ops.c:342-379): the lane's value does not depend
// on its neighbours, and the vector code's all-in-range shortcut returns what
// the blend gives such a lane. NONPOS: x is never above zero (a softmax's
// x - max; NaN allowed), so n <= 0 always holds where it matters and the
// select of g folds to a constant -- the same bits for every x with the sign
// bit set and for NaN (tests/test_expf_nonpos.py compares the two forms).
template <bool NONPOS = false>
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
    // the three results, then a select: no branch per element
    const uint32_t g = (NONPOS || n <= 0.0f) ? 0x82000000u : 0u;
    const float s1 = __uint_as_float(g + 0x7f000000u);
    const float s2 = __uint_as_float(e - g);
    const float in_range = fmaf(j, k, k), scaled = fmaf(s2, j, s2) * s1, extreme = s1 * s1;
    return !(fabsf(n) > 126.0f) ? in_range : (fabsf(n) > 192.0f ? extreme : scaled);
}

// SiLU as src/ops.c:428-440 computes it in its eight-wide body
__device__ __forceinline__ float silu(float v) {
    return v / (1.0f + ggml_v_expf(0.0f - v));
}

// ---------------------------------------------------------------------------
// wave / block reductions
// ---------------------------------------------------------------------------

// All-reduce over the 64 lanes of a wave: the four rows of 16 lanes reduce
// among themselves with DPP moves (xor 1, xor 2, half-row mirror, row
// mirror: every lane of a row then holds its row's total), and the four row
// totals are read with v_readlane. No LDS round trip, unlike a ds_bpermute
// per step. Every lane of the wave must be active.
enum : int { DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140,
             DPP_ROW_SHL4 = 0x104 };   // row_shl:4: lane i takes lane i + 4 of its row of 16

template <int CTRL>
__device__ __forceinline__ int dpp_mov(int v) { return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false); }

template <int CTRL>
__device__ __forceinline__ float dpp_mov_f(float v) { return __int_as_float(dpp_mov<CTRL>(__float_as_int(v))); }

__device__ __forceinline__ float lane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_mov_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_mov_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_mov_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_mov_f<DPP_MIRROR>(v));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_mov_u64(uint64_t v) {
    const uint32_t lo = (uint32_t) dpp_mov<CTRL>((int) (uint32_t) v);
    const uint32_t hi = (uint32_t) dpp_mov<CTRL>((int) (uint32_t) (v >> 32));
    return ((uint64_t) hi << 32) | lo;
}

__device__ __forceinline__ uint64_t lane_u64(uint64_t v, int lane) {
    const uint32_t lo = (uint32_t) __builtin_amdgcn_readlane((int) (uint32_t) v, lane);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_readlane((int) (uint32_t) (v >> 32), lane);
    return ((uint64_t) hi << 32) | lo;
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = max_u64(v, dpp_mov_u64<DPP_XOR1>(v));
    v = max_u64(v, dpp_mov_u64<DPP_XOR2>(v));
    v = max_u64(v, dpp_mov_u64<DPP_HALF_MIRROR>(v));
    v = max_u64(v, dpp_mov_u64<DPP_MIRROR>(v));
    return max_u64(max_u64(lane_u64(v, 0), lane_u64(v, 16)), max_u64(lane_u64(v, 32), lane_u64(v, 48)));
}

__device__ __forceinline__ int wave_sum(int v) {
    v += dpp_mov<DPP_XOR1>(v);
    v += dpp_mov<DPP_XOR2>(v);
    v += dpp_mov<DPP_HALF_MIRROR>(v);
    v += dpp_mov<DPP_MIRROR>(v);
    return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
           (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
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

// The slab kernel's form of chunk_dot: field 0 taken as (w ^ 0x80) & 0xC0
// in one v_bitop3 -- byte values 64 (code - 2), as signed int8 -128, -64, 0
// -- instead of a shift and a mask. Its accumulator is then 64 (D0 - 2 A0)
// for D0 the field's true dot and A0 the sum of the activation elements the
// field covers, which finish_x adds back once per row. No slot is masked:
// activation bytes past the row are zero, so whatever the weight bytes of a
// slot past the row hold, it adds nothing.
__device__ __forceinline__ void chunk_dot_x(const u32x4 wv, const int8_t *__restrict__ a, dot4acc &acc) {
    const i32x4 q0 = *reinterpret_cast<const i32x4 *>(a);
    const i32x4 q1 = *reinterpret_cast<const i32x4 *>(a + 32);
    const i32x4 q2 = *reinterpret_cast<const i32x4 *>(a + 64);
    const i32x4 q3 = *reinterpret_cast<const i32x4 *>(a + 96);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        acc.f3 = __builtin_amdgcn_sdot4((int) (wv[d] & 0x03030303u), q3[d], acc.f3, false);
        acc.f2 = __builtin_amdgcn_sdot4((int) (wv[d] & 0x0C0C0C0Cu), q2[d], acc.f2, false);
        acc.f1 = __builtin_amdgcn_sdot4((int) (wv[d] & 0x30303030u), q1[d], acc.f1, false);
        // LUT 0x28: (src0 ^ src1) & src2
        acc.f0 = __builtin_amdgcn_sdot4((int) __builtin_amdgcn_bitop3_b32(wv[d], 0x80808080u, 0xC0C0C0C0u, 0x28),
                                        q0[d], acc.f0, false);
    }
}
// one lane's share of a row's dot from chunk_dot_x's accumulators; the row's
// total is the sum over its lanes plus 2 A0
__device__ __forceinline__ int finish_x(const dot4acc &acc) {
    return acc.f3 + (acc.f2 >> 2) + (acc.f1 >> 4) + (acc.f0 >> 6);
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

// 0 in a VGPR the compiler cannot see through. A load indexed by it is a
// vector load (counted by vmcnt) even where its address is uniform: a
// uniform load of read-only memory would otherwise be a scalar load, and
// the next wait on any scalar load (lgkmcnt, which cannot tell them apart)
// would stall on its trip to HBM.
__device__ __forceinline__ uint32_t vzero() {
    uint32_t z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    return z;
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
    int     red_a[SLAB_WAVES];
};

// Every load of the slab kernel is unconditional: a skipped load (a branch
// around it, or an exec-masked block the wave jumps over when no lane needs
// it) leaves the compiler unsure how many loads are outstanding where paths
// meet, and it then waits for all of them, draining the prefetch. Weights
// are read through a buffer resource bounded by the tensor's size (the host
// keeps slab tensors at or below 0xFFFF0000 bytes): a chunk slot past the end of the last row
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

// A load that must not happen (a prefetch past the slab's last group) goes to
// this offset. The host keeps every slab tensor at or below it, so the
// resource's range check returns zeros and no memory is read.
constexpr uint32_t SLAB_DEAD_OFFSET = 0xFFFF0000u;

template <int LPR, int CPL>
__device__ __forceinline__ void slab_load(__amdgpu_buffer_rsrc_t rsrc, uint32_t row_bytes, uint32_t base,
                                          uint32_t last_row, u32x4 (&buf)[CPL], bool live = true) {
    const int lane = threadIdx.x & 63;
    const uint32_t row = min(base + (uint32_t) (lane / LPR), last_row);
    const uint32_t off = live ? row * row_bytes + (uint32_t) (lane % LPR) * 16u : SLAB_DEAD_OFFSET;
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

// slab_dot over chunk_dot_x: a2 = 2 A0 of the activation row; the LDS row
// must be zero from K to LPR * CPL * 64
template <int LPR, int CPL>
__device__ __forceinline__ void slab_dot_x(uint32_t row0, uint32_t n_rows, const u32x4 (&buf)[CPL],
                                           const int8_t *q_lds, int32_t a2, int32_t *dots) {
    const int lane = threadIdx.x & 63, sub = lane % LPR;
    const uint32_t row = row0 + (uint32_t) (lane / LPR);
    uint32_t lds_lane = (uint32_t) (sub >> 1) * 128u + (uint32_t) (sub & 1) * 16u;
    asm volatile("" : "+v"(lds_lane));
    dot4acc acc = { 0, 0, 0, 0 };
#pragma unroll
    for (int u = 0; u < CPL; ++u) chunk_dot_x(buf[u], q_lds + lds_lane + (uint32_t) (u * LPR * 64), acc);
    const int dot = group_sum<LPR>(finish_x(acc)) + a2;   // whole wave active here
    if (row < n_rows && sub == 0) dots[lane / LPR] = dot;
}


} // namespace

#endif // SLLM_I2S_DEVICE_H
