// common.hpp -- device types and helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace splosh {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kGroup = 64;       // MLX affine group size (Quant/MlxAffine.swift:22)
constexpr int kTileRows = 128;   // Converter.tileRows (Model/Retile.swift:17)

// bf16 bit pattern -> fp32: the value is the top half of the float (Q4BufferLayout.swift:123-125).
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits) {
    return __uint_as_float(bits << 16);
}

// IEEE binary16 bit pattern -> fp32 (exact widening, v_cvt_f32_f16).
__device__ __forceinline__ float half_bits_to_f32(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xffffu));
}

// fp32 -> bf16 with round-to-nearest-even (NaN stays NaN), one instruction on gfx950.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    f32x2 v = {lo, hi};
    bf16x2 r = __builtin_convertvector(v, bf16x2);
    return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float v) {
    return (uint16_t)(f32x2_to_bf16x2(v, 0.0f) & 0xffffu);
}

// The tiled record of (row n, group g) for `groups` groups a row (Model/Retile.swift:142-147).
__device__ __forceinline__ int64_t tiled_record(int64_t n, int64_t g, int64_t groups) {
    return ((n >> 7) * groups + g) * kTileRows + (n & (kTileRows - 1));
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// v_perm_b32: byte i of the result is byte sel[i] of the 8-byte value {hi, lo} (lo = bytes 0..3).
__device__ __forceinline__ uint32_t perm_bytes(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// Raw buffer access: a 128-bit resource (base, byte size) in SGPRs, a 32-bit per-lane offset and a
// wave-uniform offset, no 64-bit address arithmetic. Reads at per-lane offsets past `bytes` return
// zero; the uniform offset is kept in bounds by the callers.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 buffer_load16(rsrc_t r, uint32_t voffset, uint32_t soffset) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voffset, (int)soffset, 0);
}
// A load of streamed data (read once): the cache-policy bits of the instruction (gfx94x: sc0 = 1,
// nt = 2, sc1 = 16) as a template argument.
template <int CPOL>
__device__ __forceinline__ u32x4 buffer_load16_cp(rsrc_t r, uint32_t voffset, uint32_t soffset) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voffset, (int)soffset, CPOL);
}
__device__ __forceinline__ uint32_t buffer_load_u32(rsrc_t r, uint32_t voffset, uint32_t soffset) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voffset, (int)soffset, 0);
}
__device__ __forceinline__ uint32_t buffer_load_u16(rsrc_t r, uint32_t voffset, uint32_t soffset) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)voffset, (int)soffset, 0);
}

// 16 bytes a lane from a buffer straight into LDS (the load's LDS modifier, gfx950): lane l of
// the wave writes bytes [16 l, 16 l + 16) after `lds_dst`, which must be wave-uniform. The load
// counts in vmcnt; once it has been waited for, the data is in LDS. (The host pass compiles no
// kernel code, and has no LDS address space, hence the guard.)
__device__ __forceinline__ void buffer_load_lds16(rsrc_t r, void *lds_dst, uint32_t voffset) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds_dst, 16, (int)voffset, 0, 0, 0);
#else
    (void)r, (void)lds_dst, (void)voffset;
#endif
}

// 4 bytes a lane straight into LDS: lane l writes bytes [4 l, 4 l + 4) after `lds_dst`
// (wave-uniform), as buffer_load_lds16.
__device__ __forceinline__ void buffer_load_lds4(rsrc_t r, void *lds_dst, uint32_t voffset) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds_dst, 4, (int)voffset, 0, 0, 0);
#else
    (void)r, (void)lds_dst, (void)voffset;
#endif
}

// s_waitcnt with only vmcnt bounded (expcnt and lgkmcnt left at their maxima), gfx9 encoding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS operations, not for its
// outstanding global loads (which __syncthreads' fence would drain), so prefetches stay in flight.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// lds_barrier() at a hand-off where up to OUTSTANDING loads into LDS, the youngest ones issued,
// are meant to stay in flight. The count is written into the assembly as a comment, where a
// static check compares it with what the preceding vmcnt wait really leaves outstanding.
template <int OUTSTANDING>
__device__ __forceinline__ void lds_barrier_staged() {
    asm volatile("; splosh-lds-outstanding %0\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(OUTSTANDING) : "memory");
}

// The block a workgroup takes when neighbouring blocks share cache lines: workgroups are handed to
// the eight XCDs (each with its own L2) round robin by id, so consecutive ids land on different
// L2s and a line two neighbours share is fetched from memory twice. Block = (id mod 8) (G / 8) +
// id / 8 gives every XCD a contiguous run of blocks instead (G a multiple of 8; otherwise the id
// itself). Only the order of the work changes.
__device__ __forceinline__ int xcd_block(int id, int grid) {
    return grid % 8 == 0 ? (id & 7) * (grid >> 3) + (id >> 3) : id;
}

// The activation group (32 elements) that weight group g meets when the weight's inner columns keep
// a GGUF file's order of the gated-delta value heads (128 columns, four groups, each) and the
// activations the engine's (engine_gguf.metal:55-72, GgufNames.swift mlxValueHead): file head h is
// engine head vph (h mod kh) + h / kh, kh = 2^hs key heads, vph value heads each. hs < 0: no
// reordering.
__device__ __forceinline__ int head_group(int g, int hs, int vph) {
    if (hs < 0) return g;
    const int head = g >> 2;
    return ((vph * (head & ((1 << hs) - 1)) + (head >> hs)) << 2) | (g & 3);
}

// Byte j of x as an fp32 number (v_cvt_f32_ubyteN, exact).
__device__ __forceinline__ float cvt_byte(uint32_t x, int j) {
    float r;
    switch (j) {
        case 0: asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(x)); break;
        case 1: asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(x)); break;
        case 2: asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(x)); break;
        default: asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(x)); break;
    }
    return r;
}

// x sigmoid(x) with the hardware reciprocal (v_rcp_f32, about 1 ulp) instead of a full-precision
// divide: the result is rounded to bf16 or summed in fp32 afterwards.
__device__ __forceinline__ float silu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// ---- Balance split of a streaming kernel's last round -----------------------------------------
//
// A kernel whose workgroups each own a block of output rows over all of K runs as long as the CUs
// that hold one block more than the others. When the blocks do not divide evenly over the CUs,
// the whole rounds stay whole and each block of the last round is cut into `slices` ranges of K
// units, one workgroup a slice, so that every CU holds its whole blocks and one slice. A slice
// writes its fp32 sums to a workspace and counts itself in on the block's arrival counter; the
// last to arrive adds the partials in slice order (the result does not depend on who arrives
// last) and writes the rows.

struct BalanceSplit {
    int nwhole, tail, slices;  // slices < 2: every block whole
};
constexpr int kBalanceMaxSlices = 16;
// The workspace's first 16 KiB hold the arrival counters (zero between calls, the region every
// kernel's counters share); the partials follow.
constexpr size_t kBalanceCounterBytes = 16384;

// The split for `blocks` row blocks of `units` units of K on `cus` CUs: only where every CU
// already holds two whole blocks or more, and the whole blocks and the slices divide by 8 (the
// XCD interleave of balance_block).
inline BalanceSplit plan_balance(int64_t blocks, int cus, int units) {
    const int64_t base = blocks / cus * cus, tail = blocks - base;
    BalanceSplit p{(int)blocks, 0, 1};
    if (base < 2 * (int64_t)cus || tail == 0 || base % 8 != 0) return p;
    int slices = (int)(cus / tail);
    slices = slices < units ? slices : units;
    slices = slices < kBalanceMaxSlices ? slices : kBalanceMaxSlices;
    while (slices >= 2 && (tail * slices) % 8 != 0) --slices;
    if (slices >= 2) p = BalanceSplit{(int)base, (int)tail, slices};
    return p;
}

// Workgroup `id` of the split grid: its block and units [ua, ub); tb >= 0 (and its slice sl) for a
// slice of tail block tb. Workgroup i goes to XCD i mod 8, and each XCD takes the same share of
// whole blocks (contiguous, as xcd_block) and of slices. Without a split, xcd_block's order.
__device__ __forceinline__ void balance_block(int id, int grid, int nwhole, int tail, int slices, int units, int &blk,
                                              int &ua, int &ub, int &tb, int &sl) {
    ua = 0;
    ub = units;
    tb = -1;
    sl = 0;
    if (slices < 2) {
        blk = xcd_block(id, grid);
        return;
    }
    const int x = id & 7, j = id >> 3;
    const int wpx = nwhole >> 3;  // whole blocks an XCD
    if (j < wpx) {
        blk = x * wpx + j;
        return;
    }
    const int q = x * ((tail * slices) >> 3) + (j - wpx);
    tb = q / slices;
    sl = q - tb * slices;
    blk = nwhole + tb;
    ua = (int)((int64_t)units * sl / slices);
    ub = (int)((int64_t)units * (sl + 1) / slices);
}

// The merge of a slice's NV values a thread (threads [0, nact) hold values): written through to
// memory (gfx94x cache policy sc0 sc1: the summing workgroup may run on another XCD, whose L2 is
// not coherent with this one's), then the arrival. Returns true for the last slice to arrive,
// with `v` replaced by the sums over all slices in slice order. Every thread of the workgroup
// calls it.
template <int NV>
__device__ __forceinline__ bool balance_merge(float (&v)[NV], int tid, int nact, int tb, int sl, int slices,
                                              float *partial, uint32_t partial_bytes, int *counters) {
    constexpr int kCpol = 1 | 16;
    const rsrc_t p_rsrc = make_rsrc(partial, partial_bytes);
    auto off = [&](int slice, int j) { return (uint32_t)((((tb * slices + slice) * NV + j) * nact + tid) * 4); };
    if (tid < nact) {
#pragma unroll
        for (int j = 0; j < NV; ++j)
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v[j]), p_rsrc, off(sl, j), 0, kCpol);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial is in memory
    __syncthreads();
    __shared__ int arrival;
    if (tid == 0) {
        const int old = __hip_atomic_fetch_add(counters + tb, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        if (old == slices - 1) __hip_atomic_store(counters + tb, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        arrival = old;
    }
    __syncthreads();
    if (arrival != slices - 1) return false;
    if (tid < nact) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            // Every slice's partial loaded first (one round trip), then added in slice order.
            float part[kBalanceMaxSlices];
#pragma unroll
            for (int q = 0; q < kBalanceMaxSlices; ++q)
                part[q] = q < slices ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(p_rsrc, off(q, j), 0, kCpol))
                                     : 0.0f;
            float sum = 0.0f;
#pragma unroll
            for (int q = 0; q < kBalanceMaxSlices; ++q)
                if (q < slices) sum += part[q];
            v[j] = sum;
        }
    }
    return true;
}

}  // namespace splosh
