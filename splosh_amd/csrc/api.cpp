// api.cpp -- the C ABI (include/splosh_q4.h): argument validation with the reference's error
// semantics, the kernel-choice policy, and launches. Everything here is host code; it never
// allocates device memory and never synchronises a stream.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>

#include "../../include/splosh_q4.h"
#include "launch.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int status, const std::string &message) {
    g_last_error = message;
    return status;
}

int ok() {
    g_last_error.clear();
    return SPLOSH_OK;
}

int hip_status(hipError_t err, const char *what) {
    if (err != hipSuccess)
        return fail(SPLOSH_ERR_HIP, std::string(what) + ": " + hipGetErrorString(err));
    return ok();
}

bool mul_overflows(int64_t a, int64_t b) { return a != 0 && b > INT64_MAX / a; }

bool aligned(const void *p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

constexpr int64_t kGroupSize = 64;
constexpr int64_t kWordBytes = 4;
constexpr int64_t kDefaultRowAlignment = 128;

// Shared checks of the GEMM entry points on a q4 weight (the geometry GemmQ4Shape.validate and
// Converter.isTiledWeight require, Model/Gemm.swift:19-40, Model/Retile.swift:33-36).
int check_q4_weight(const splosh_q4_weight *w, const char *name) {
    if (!w || !w->packed || !w->scales || !w->biases)
        return fail(SPLOSH_ERR_NULL_POINTER, std::string(name) + ": null weight pointer");
    if (w->rows <= 0 || w->inner <= 0)
        return fail(SPLOSH_ERR_INVALID_SHAPE, std::string(name) + ": rows and inner must be positive");
    if (w->inner > INT64_MAX - 63) return fail(SPLOSH_ERR_INVALID_SHAPE, "inner overflows");
    if (w->order == SPLOSH_Q4_ROW_MAJOR) {
        if (w->row_stride_words < (w->inner + 7) / 8)
            return fail(SPLOSH_ERR_INVALID_ROW_STRIDE,
                        std::string(name) + ": row_stride_words is shorter than the packed row");
        if (mul_overflows(w->rows, w->row_stride_words))
            return fail(SPLOSH_ERR_ARITHMETIC_OVERFLOW, "packed size overflows");
    } else if (w->order == SPLOSH_Q4_TILED128) {
        if (w->rows % 128 != 0 || w->inner % kGroupSize != 0)
            return fail(SPLOSH_ERR_LAYOUT_MISMATCH,
                        std::string(name) + ": the tiled layout needs rows % 128 == 0 and inner % 64 == 0");
    } else {
        return fail(SPLOSH_ERR_LAYOUT_MISMATCH, std::string(name) + ": unknown weight order");
    }
    return SPLOSH_OK;
}

int check_io(const uint16_t *a, int64_t lda, const void *out, int64_t ldc, int out_dtype, int64_t rows,
             int64_t n, int64_t k) {
    if (!a || !out) return fail(SPLOSH_ERR_NULL_POINTER, "null activation or output pointer");
    if (rows <= 0) return fail(SPLOSH_ERR_INVALID_SHAPE, "rows must be positive");
    if (lda < k) return fail(SPLOSH_ERR_INVALID_SHAPE, "lda is shorter than inner");
    if (ldc < n) return fail(SPLOSH_ERR_INVALID_SHAPE, "ldc is shorter than the weight's rows");
    if (out_dtype != SPLOSH_F32 && out_dtype != SPLOSH_BF16) return fail(SPLOSH_ERR_UNSUPPORTED, "unknown out_dtype");
    if (mul_overflows(rows, lda) || mul_overflows(rows, ldc)) return fail(SPLOSH_ERR_ARITHMETIC_OVERFLOW, "size overflows");
    return SPLOSH_OK;
}

// Whether the streaming kernels can take this call: whole 64-groups, 16-byte aligned activation
// rows, 8-byte aligned code records.
bool q4_stream_eligible(const splosh_q4_weight &w, const uint16_t *a, int64_t lda) {
    if (w.inner % kGroupSize != 0) return false;
    if (lda % 8 != 0 || !aligned(a, 16)) return false;
    if (!aligned(w.packed, 8)) return false;
    if (w.order == SPLOSH_Q4_ROW_MAJOR && w.row_stride_words % 2 != 0) return false;
    return true;
}

int q4_gemm_impl(const splosh_q4_weight *w, const splosh_q4_weight *up, const uint16_t *a, int64_t lda, void *out,
                 int64_t ldc, int out_dtype, const void *residual, int64_t rows, int kernel, void *workspace,
                 size_t workspace_bytes, hipStream_t stream, const splosh::EmitOperand *emit = nullptr,
                 bool *emitted = nullptr) {
    int st = check_q4_weight(w, up ? "gate" : "weight");
    if (st) return st;
    if (up) {
        if ((st = check_q4_weight(up, "up"))) return st;
        if (up->rows != w->rows || up->inner != w->inner || up->order != w->order ||
            (w->order == SPLOSH_Q4_ROW_MAJOR && up->row_stride_words != w->row_stride_words))
            return fail(SPLOSH_ERR_LAYOUT_MISMATCH, "gate and up weights differ in geometry");
    }
    if ((st = check_io(a, lda, out, ldc, out_dtype, rows, w->rows, w->inner))) return st;
    const bool eligible = q4_stream_eligible(*w, a, lda) && (!up || q4_stream_eligible(*up, a, lda));
    const bool wide16 = eligible && aligned(w->packed, 16) && (!up || aligned(up->packed, 16)) &&
                        (w->order == SPLOSH_Q4_TILED128 || w->row_stride_words % 4 == 0);
    // 65..128 rows under AUTO: rows 0..63 and the rest as two calls of the M <= 64 kernels, one after
    // the other on the stream (the workspace's counters are zero again between them). Measured at
    // K5120 -> 2 x N17408 (gate+up) and K17408 -> N5120, against the one call on the tile or
    // prefill kernel: gate+up M=65 91 -> 60 us, M=96 94 -> 72, M=128 97 -> 80; down M=65 54 -> 38,
    // M=96 55 -> 47, M=128 58 -> 51; at 192 rows three calls lose (120 against 104 us).
    if (kernel == SPLOSH_KERNEL_AUTO && !emit && rows > 64 && rows <= 128 && wide16 &&
        splosh::mma_fits(64, w->rows, w->inner, w->row_stride_words, lda)) {
        const char *res = (const char *)residual;
        const size_t esize = out_dtype == SPLOSH_F32 ? 4 : 2;
        if ((st = q4_gemm_impl(w, up, a, lda, out, ldc, out_dtype, residual, 64, kernel, workspace, workspace_bytes,
                               stream)))
            return st;
        return q4_gemm_impl(w, up, a + 64 * lda, lda, (char *)out + 64 * ldc * esize, ldc, out_dtype,
                            res ? res + 64 * ldc * esize : nullptr, rows - 64, kernel, workspace, workspace_bytes,
                            stream);
    }
    const bool tile_ok = wide16 && splosh::tile_fits(rows, w->rows, lda, w->row_stride_words);
    const bool mma_ok = wide16 && splosh::mma_fits(rows, w->rows, w->inner, w->row_stride_words, lda);
    const bool prefill_ok = wide16 && !up && w->order == SPLOSH_Q4_TILED128 && aligned(out, 16) &&
                            (!residual || aligned(residual, 16)) &&
                            splosh::prefill_fits(rows, w->rows, w->inner, lda, ldc);
    const bool prefill_mlp_ok = wide16 && up && w->order == SPLOSH_Q4_TILED128 && up->order == SPLOSH_Q4_TILED128 &&
                                aligned(out, 16) && splosh::prefill_fits(rows, w->rows, w->inner, lda, ldc);
    const bool decode_ok = wide16 && splosh::decode_fits(rows, w->rows, w->inner, w->order);
    int choice = kernel;
    if (choice == SPLOSH_KERNEL_AUTO) {
        if (!eligible) choice = SPLOSH_KERNEL_SCALAR;
        else if (decode_ok) choice = SPLOSH_KERNEL_STREAM;
        else if (wide16 && splosh::lanes_fit(rows, w->rows, w->inner, w->row_stride_words, up != nullptr))
            choice = SPLOSH_KERNEL_STREAM;
        else if (mma_ok) choice = SPLOSH_KERNEL_DEQUANT;
        // One weight at 65..128 rows: the tile kernel where the prefill kernel's 256-row tiles are
        // mostly padding and its tiles few (measured at M=64..128: K17408 -> N5120 tile 51-56 us,
        // prefill 59-65; K5120 -> N17408 tile better at 65 rows, prefill from 96).
        else if (tile_ok && !up && rows <= 128 && (rows <= 80 || w->rows <= 8192)) choice = SPLOSH_KERNEL_TILE;
        else if (prefill_ok || prefill_mlp_ok) choice = SPLOSH_KERNEL_PREFILL;
        else if (tile_ok) choice = SPLOSH_KERNEL_TILE;
        else choice = SPLOSH_KERNEL_STREAM;
    }
    switch (choice) {
        case SPLOSH_KERNEL_PREFILL: {
            if (prefill_mlp_ok) {
                const splosh::PrefillPlan plan =
                    splosh::plan_prefill(rows, 2 * w->rows, w->inner / kGroupSize, workspace ? workspace_bytes : 0);
                return hip_status(splosh::launch_q4_prefill_mlp(plan, *w, *up, a, lda, out, ldc, out_dtype, rows,
                                                                workspace, stream),
                                  "q4 prefill gate+up launch");
            }
            if (!prefill_ok)
                return fail(SPLOSH_ERR_UNSUPPORTED,
                            "prefill kernel needs one TILED128 weight, lda % 8 == 0, ldc % 4 == 0 and 16-byte "
                            "aligned operands");
            const splosh::PrefillPlan plan =
                splosh::plan_prefill(rows, w->rows, w->inner / kGroupSize, workspace ? workspace_bytes : 0);
            if (emitted) *emitted = emit != nullptr;
            return hip_status(splosh::launch_q4_prefill(plan, *w, a, lda, out, ldc, out_dtype, residual, rows,
                                                        workspace, stream, emit),
                              "q4 prefill launch");
        }
        case SPLOSH_KERNEL_TILE: {
            if (!tile_ok)
                return fail(SPLOSH_ERR_UNSUPPORTED,
                            "tile kernel needs inner % 64 == 0, lda % 8 == 0, 16-byte aligned operands and "
                            "32-bit element offsets");
            const splosh::TilePlan plan =
                splosh::plan_tile(rows, w->rows, w->inner / kGroupSize, up != nullptr, workspace ? workspace_bytes : 0);
            return hip_status(splosh::launch_q4_tile(plan, *w, up, a, lda, out, ldc, out_dtype, residual, rows,
                                                     workspace, stream),
                              "q4 tile launch");
        }
        case SPLOSH_KERNEL_STREAM: {
            if (!eligible)
                return fail(SPLOSH_ERR_UNSUPPORTED,
                            "stream kernel needs inner % 64 == 0, lda % 8 == 0 and aligned operands");
            if (wide16 && decode_ok) {
                return hip_status(splosh::launch_q4_decode(*w, up, a, lda, out, ldc, out_dtype, residual, rows,
                                                           workspace, workspace ? workspace_bytes : 0, stream),
                                  "q4 decode launch");
            }
            if (wide16 && splosh::lanes_fit(rows, w->rows, w->inner, w->row_stride_words, up != nullptr)) {
                const splosh::StreamPlan plan = splosh::plan_lanes(rows, w->rows, w->inner / kGroupSize, up != nullptr);
                return hip_status(splosh::launch_q4_lanes(plan, *w, up, a, lda, out, ldc, out_dtype, residual, rows,
                                                          stream),
                                  "q4 lanes launch");
            }
            const splosh::StreamPlan plan = splosh::plan_stream(rows, w->rows, w->inner / kGroupSize, up != nullptr, 4);
            if (plan.row_chunks > 65535) return fail(SPLOSH_ERR_UNSUPPORTED, "too many rows for one launch");
            return hip_status(splosh::launch_q4_stream(plan, *w, up, a, lda, out, ldc, out_dtype, residual, rows, stream),
                              "q4 stream launch");
        }
        case SPLOSH_KERNEL_SCALAR:
            if (rows > 65535) return fail(SPLOSH_ERR_UNSUPPORTED, "scalar kernel takes at most 65535 rows");
            return hip_status(splosh::launch_q4_gemm_scalar(*w, up, a, lda, out, ldc, out_dtype, residual, rows, stream),
                              "q4 scalar launch");
        case SPLOSH_KERNEL_DEQUANT: {
            if (!mma_ok) return fail(SPLOSH_ERR_UNSUPPORTED, "dequant kernel needs rows <= 64 and aligned operands");
            // The emit epilogue only when asked for by name: under AUTO the GEMM plus the separate
            // pass is the faster of the two at these row counts.
            const splosh::EmitOperand *mma_emit = kernel == SPLOSH_KERNEL_DEQUANT ? emit : nullptr;
            if (emitted) *emitted = mma_emit != nullptr;
            // A wide single weight: its two column halves as a pair.
            const bool split = !up && !mma_emit && splosh::mma_split(*w);
            const splosh::MmaPlan plan = splosh::plan_mma(rows, split ? w->rows / 2 : w->rows, w->inner / kGroupSize,
                                                          up != nullptr || split, workspace ? workspace_bytes : 0);
            if (split)
                return hip_status(splosh::launch_q4_mma_split(plan, *w, a, lda, out, ldc, out_dtype, residual, rows,
                                                              workspace, stream),
                                  "q4 mma launch");
            return hip_status(splosh::launch_q4_mma(plan, *w, up, a, lda, out, ldc, out_dtype, residual, rows,
                                                    workspace, stream, mma_emit),
                              "q4 mma launch");
        }
        default:
            return fail(SPLOSH_ERR_UNSUPPORTED, "unknown kernel choice");
    }
}

// fifth = false: Q4_K planes (no plane1).
int check_q5k_weight(const splosh_q5k_weight *w, bool fifth = true) {
    if (!w || !w->plane0 || (fifth && !w->plane1) || !w->meta) return fail(SPLOSH_ERR_NULL_POINTER, "null GGUF plane pointer");
    if (w->rows <= 0 || w->inner <= 0) return fail(SPLOSH_ERR_INVALID_SHAPE, "rows and inner must be positive");
    // GgufPlanes.sizes: whole tiles of 128 rows, whole 256-element blocks (GgufPlanes.swift:78-86).
    if (w->rows % 128 != 0 || w->inner % 256 != 0)
        return fail(SPLOSH_ERR_LAYOUT_MISMATCH, "Q5_K planes need rows % 128 == 0 and inner % 256 == 0");
    return SPLOSH_OK;
}

// ---- the allocation-free entry point's scratch ------------------------------------------------
//
// splosh_q4_gemm_noalloc runs the same kernels as splosh_q4_gemm with this file-scope device array
// as its workspace: the split-K arrival counters (first 16 KiB, as in any workspace) and the
// partials of the M <= 64 MFMA kernel on one weight (grid x 2 slots x 64 rows x 64 columns fp32 =
// 8 MiB at the 256 workgroups of an MI355X). Every GPU the library runs on holds its own copy
// until the process ends. In host code `scratch` names a host-side stand-in, never the device
// memory: its address on each device comes from hipGetSymbolAddress, once per device.
constexpr size_t kScratchBytes = (size_t)16384 + ((size_t)8 << 20);
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices] = {nullptr};

// The scratch array's device address on the current device (looked up on the first call there).
int scratch_on_current_device(void **out) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return fail(SPLOSH_ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(err));
    if (dev < 0 || dev >= kMaxDevices) return fail(SPLOSH_ERR_UNSUPPORTED, "device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err != hipSuccess || !ptr)
            return fail(SPLOSH_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(err));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return SPLOSH_OK;
}

// Zeroes `words` 32-bit words (a fill kernel rather than hipMemsetAsync, so that a caller may
// capture the call in a HIP graph).
__global__ void zero_words_kernel(uint32_t *p, int words) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < words; i += gridDim.x * blockDim.x) p[i] = 0u;
}

}  // namespace

extern "C" {

const char *splosh_version(void) { return "splosh-amd 0.1.0 (gfx950)"; }

const char *splosh_last_error(void) { return g_last_error.c_str(); }

const char *splosh_status_string(int status) {
    switch (status) {
        case SPLOSH_OK: return "ok";
        case SPLOSH_ERR_INVALID_SHAPE: return "invalidShape";
        case SPLOSH_ERR_LAYOUT_MISMATCH: return "layoutMismatch";
        case SPLOSH_ERR_INVALID_ROW_STRIDE: return "invalidRowStride";
        case SPLOSH_ERR_ORIENTATION_MISMATCH: return "orientationMismatch";
        case SPLOSH_ERR_INVALID_GROUP_SIZE: return "invalidGroupSize";
        case SPLOSH_ERR_SIDECAR_GEOMETRY_MISMATCH: return "sidecarGeometryMismatch";
        case SPLOSH_ERR_SIDECAR_MISMATCH: return "sidecarMismatch";
        case SPLOSH_ERR_BUFFER_TOO_SMALL: return "bufferTooSmall";
        case SPLOSH_ERR_INVALID_DIMENSIONS: return "invalidDimensions";
        case SPLOSH_ERR_ARITHMETIC_OVERFLOW: return "arithmeticOverflow";
        case SPLOSH_ERR_INVALID_INDEX: return "invalidIndex";
        case SPLOSH_ERR_NULL_POINTER: return "nullPointer";
        case SPLOSH_ERR_UNSUPPORTED: return "unsupported";
        case SPLOSH_ERR_WORKSPACE_TOO_SMALL: return "workspaceTooSmall";
        case SPLOSH_ERR_HIP: return "hipError";
        default: return "unknown";
    }
}

// Q4BufferLayout.init (Quant/Q4BufferLayout.swift:43-79).
int splosh_q4_layout_init(int64_t rows, int64_t logical_k, int orientation, int64_t row_stride_bytes,
                          int64_t row_alignment, splosh_q4_layout *out) {
    if (!out) return fail(SPLOSH_ERR_NULL_POINTER, "null layout");
    if (row_alignment == 0) row_alignment = kDefaultRowAlignment;
    if (rows <= 0 || logical_k <= 0 || row_alignment <= 0 ||
        (orientation != SPLOSH_ROWS_BY_K && orientation != SPLOSH_K_BY_COLUMNS))
        return fail(SPLOSH_ERR_INVALID_DIMENSIONS, "rows, logical_k and alignment must be positive");
    if (logical_k > INT64_MAX - 7 || rows > INT64_MAX - 7) return fail(SPLOSH_ERR_ARITHMETIC_OVERFLOW, "overflow");
    const int64_t packed = orientation == SPLOSH_ROWS_BY_K ? (logical_k + 7) / 8 : (rows + 7) / 8;
    if (packed > INT64_MAX / kWordBytes) return fail(SPLOSH_ERR_ARITHMETIC_OVERFLOW, "overflow");
    const int64_t minimum = packed * kWordBytes;
    int64_t stride;
    if (row_stride_bytes != 0) {
        stride = row_stride_bytes;
    } else {
        if (minimum > INT64_MAX - row_alignment + 1) return fail(SPLOSH_ERR_ARITHMETIC_OVERFLOW, "overflow");
        const int64_t blocks = (minimum + row_alignment - 1) / row_alignment;
        if (blocks > INT64_MAX / row_alignment) return fail(SPLOSH_ERR_ARITHMETIC_OVERFLOW, "overflow");
        stride = blocks * row_alignment;
    }
    if (stride < minimum || stride % kWordBytes != 0)
        return fail(SPLOSH_ERR_INVALID_ROW_STRIDE, "row stride is shorter than the row or not whole words");
    if (logical_k > INT64_MAX - (kGroupSize - 1)) return fail(SPLOSH_ERR_ARITHMETIC_OVERFLOW, "overflow");
    const int64_t groups = (logical_k + kGroupSize - 1) / kGroupSize;
    const int64_t physical_rows = orientation == SPLOSH_ROWS_BY_K ? rows : logical_k;
    if (physical_rows > INT64_MAX / (stride / kWordBytes) || rows > INT64_MAX / groups)
        return fail(SPLOSH_ERR_ARITHMETIC_OVERFLOW, "overflow");
    out->rows = rows;
    out->logical_k = logical_k;
    out->orientation = orientation;
    out->reserved = 0;
    out->packed_words_per_row = packed;
    out->row_stride_bytes = stride;
    out->row_stride_words = stride / kWordBytes;
    out->padding_words_per_row = stride / kWordBytes - packed;
    out->groups_per_row = groups;
    out->group_stride = groups;
    return ok();
}

static int validate_index(const splosh_q4_layout *l, int64_t row, int64_t k) {
    if (!l) return fail(SPLOSH_ERR_NULL_POINTER, "null layout");
    if (row < 0 || row >= l->rows || k < 0 || k >= l->logical_k)
        return fail(SPLOSH_ERR_INVALID_INDEX, "index out of the logical matrix");
    return SPLOSH_OK;
}

// Q4BufferLayout.wordIndex (Q4BufferLayout.swift:82-92).
int splosh_q4_layout_word_index(const splosh_q4_layout *l, int64_t row, int64_t k, int64_t *out) {
    int st = validate_index(l, row, k);
    if (st) return st;
    if (!out) return fail(SPLOSH_ERR_NULL_POINTER, "null output");
    *out = l->orientation == SPLOSH_ROWS_BY_K ? row * l->row_stride_words + k / 8 : k * l->row_stride_words + row / 8;
    return ok();
}

// Q4BufferLayout.nibbleShift (Q4BufferLayout.swift:94-98).
int splosh_q4_layout_nibble_shift(const splosh_q4_layout *l, int64_t row, int64_t k, uint32_t *out) {
    int st = validate_index(l, row, k);
    if (st) return st;
    if (!out) return fail(SPLOSH_ERR_NULL_POINTER, "null output");
    *out = (uint32_t)((l->orientation == SPLOSH_ROWS_BY_K ? k % 8 : row % 8) * 4);
    return ok();
}

// Q4BufferLayout.sidecarIndex (Q4BufferLayout.swift:100-104).
int splosh_q4_layout_sidecar_index(const splosh_q4_layout *l, int64_t row, int64_t k, int64_t *out) {
    int st = validate_index(l, row, k);
    if (st) return st;
    if (!out) return fail(SPLOSH_ERR_NULL_POINTER, "null output");
    *out = row * l->group_stride + k / kGroupSize;
    return ok();
}

// GemmQ4Shape.init + validate(layout:) (Model/Gemm.swift:13-40).
int splosh_q4_shape_validate(int64_t rows, int64_t columns, int64_t inner, const splosh_q4_layout *l) {
    if (rows <= 0 || columns <= 0 || inner <= 0) return fail(SPLOSH_ERR_INVALID_SHAPE, "invalidShape");
    if (!l) return fail(SPLOSH_ERR_NULL_POINTER, "null layout");
    if (l->rows != columns || l->logical_k != inner) return fail(SPLOSH_ERR_LAYOUT_MISMATCH, "layoutMismatch");
    if (l->orientation != SPLOSH_ROWS_BY_K) return fail(SPLOSH_ERR_ORIENTATION_MISMATCH, "orientationMismatch");
    if (l->row_stride_bytes < kDefaultRowAlignment || l->row_stride_bytes % kDefaultRowAlignment != 0 ||
        l->row_stride_bytes % kWordBytes != 0 || l->row_stride_bytes < l->packed_words_per_row * kWordBytes)
        return fail(SPLOSH_ERR_INVALID_ROW_STRIDE, "invalidRowStride");
    if (inner > INT64_MAX - (kGroupSize - 1)) return fail(SPLOSH_ERR_INVALID_SHAPE, "invalidShape");
    if (l->groups_per_row != (inner + kGroupSize - 1) / kGroupSize || l->group_stride != l->groups_per_row)
        return fail(SPLOSH_ERR_SIDECAR_GEOMETRY_MISMATCH, "sidecarGeometryMismatch");
    return ok();
}

size_t splosh_workspace_bytes(int64_t rows, int64_t columns, int64_t inner) {
    if (rows <= 0 || columns <= 0 || inner < kGroupSize) return 0;
    const int64_t groups = inner / kGroupSize;
    const size_t tile = splosh::tile_workspace_bytes(rows, columns, groups, true);
    // (65..128 rows run as two calls of at most 64 rows.)
    const size_t mma = rows <= 128 ? splosh::mma_workspace_bytes(rows < 64 ? rows : 64, columns, groups, true) : 0;
    // (2 columns: the fused gate+up plans its tiles over both weights' columns.)
    const size_t prefill = rows > 64 && columns % 128 == 0 ? splosh::prefill_workspace_bytes(rows, 2 * columns, groups) : 0;
    const size_t gguf = inner % 64 == 0 ? splosh::gguf_tile_workspace_bytes(rows, columns, inner) : 0;
    const size_t decode = splosh::decode_workspace_bytes(rows, columns, inner, 2);
    const size_t q5k_decode = splosh::q5k_decode_workspace_bytes(rows, columns, inner);
    size_t need = tile > mma ? tile : mma;
    need = need > decode ? need : decode;
    need = need > q5k_decode ? need : q5k_decode;
    need = need > prefill ? need : prefill;
    return need > gguf ? need : gguf;
}

// Q4GemmRuntime.dispatch (Runtime/Q4Runtime.swift:94-145).
int splosh_gemm_q4(const uint16_t *a, const uint32_t *packed, const uint16_t *scales, const uint16_t *biases,
                   float *c, int64_t rows, int64_t columns, int64_t inner, const splosh_q4_layout *layout,
                   hipStream_t stream) {
    int st = splosh_q4_shape_validate(rows, columns, inner, layout);
    if (st) return st;
    if (mul_overflows(rows, inner) || mul_overflows(rows, columns) || rows > 65535)
        return fail(SPLOSH_ERR_INVALID_SHAPE, "invalidShape");
    if (!a || !packed || !scales || !biases || !c) return fail(SPLOSH_ERR_NULL_POINTER, "null buffer");
    return hip_status(splosh::launch_gemm_q4_scalar(a, packed, scales, biases, c, rows, columns, inner,
                                                    layout->row_stride_words, layout->orientation,
                                                    layout->groups_per_row, stream),
                      "gemm_q4 launch");
}

int splosh_q4_gemm(const splosh_q4_weight *w, const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                   const void *residual, int64_t rows, int kernel, void *workspace, size_t workspace_bytes,
                   hipStream_t stream) {
    return q4_gemm_impl(w, nullptr, a, lda, out, ldc, out_dtype, residual, rows, kernel, workspace, workspace_bytes,
                        stream);
}

// Engine.gemm with emit (engine_na.metal:322-473): the residual projection that also writes the
// next RMSNorm's operand. The prefill kernel (AUTO from 256 rows for most shapes) writes it from its
// epilogue, and so does the M <= 64 kernel when SPLOSH_KERNEL_DEQUANT is asked for; otherwise the
// GEMM is followed by the separate operand pass on the fp32 output (at M=64, K17408 -> N5120 the
// GEMM plus the pass takes 30.1 us, the fused M <= 64 epilogue 31.2 us).
int splosh_q4_gemm_emit(const splosh_q4_weight *w, const uint16_t *a, int64_t lda, float *out, int64_t ldc,
                        const float *residual, int64_t rows, const uint16_t *norm_weight, uint16_t *values,
                        int64_t ld_values, float *sums, float *squares, int kernel, void *workspace,
                        size_t workspace_bytes, hipStream_t stream) {
    int st = check_q4_weight(w, "weight");
    if (st) return st;
    if (!norm_weight || !values || !sums || !squares) return fail(SPLOSH_ERR_NULL_POINTER, "null emit buffer");
    if (w->rows % 64 != 0) return fail(SPLOSH_ERR_INVALID_SHAPE, "emit needs the output width to be a multiple of 64");
    if (ld_values < w->rows) return fail(SPLOSH_ERR_INVALID_SHAPE, "ld_values is shorter than the output width");
    if (!aligned(out, 16) || ldc % 4 != 0 || !aligned(values, 8) || ld_values % 4 != 0 || !aligned(norm_weight, 8))
        return fail(SPLOSH_ERR_UNSUPPORTED,
                    "emit needs a 16-byte aligned fp32 output with ldc % 4 == 0, 8-byte aligned values with "
                    "ld_values % 4 == 0 and an 8-byte aligned norm weight");
    const splosh::EmitOperand emit{norm_weight, values, ld_values, sums, squares};
    bool emitted = false;
    if ((st = q4_gemm_impl(w, nullptr, a, lda, out, ldc, SPLOSH_F32, residual, rows, kernel, workspace,
                           workspace_bytes, stream, &emit, &emitted)))
        return st;
    if (emitted) return ok();
    return hip_status(splosh::launch_emit_operand(out, ldc, norm_weight, rows, w->rows, values, ld_values, sums, squares,
                                                  stream),
                      "emit operand launch");
}

// splosh_q4_gemm with the library's static device scratch as its workspace: no allocation.
int splosh_q4_gemm_noalloc(const splosh_q4_weight *w, const uint16_t *a, int64_t lda, void *out, int64_t ldc,
                           int out_dtype, const void *residual, int64_t rows, int kernel, hipStream_t stream) {
    int st = check_q4_weight(w, "weight");
    if (st) return st;
    if ((st = check_io(a, lda, out, ldc, out_dtype, rows, w->rows, w->inner))) return st;
    // Every kernel plans against the scratch's size: one whose partials do not fit runs unsplit
    // (the M <= 64 kernel one workgroup a band, the split-K kernels with one slice).
    void *ptr = nullptr;
    if ((st = scratch_on_current_device(&ptr))) return st;
    // The arrival counters must start at zero: every call returns them to zero, and this call
    // clears them first anyway (a call that failed half-way may have left them set).
    hipLaunchKernelGGL(zero_words_kernel, dim3(4), dim3(256), 0, stream, (uint32_t *)ptr, 16384 / 4);
    if ((st = hip_status(hipGetLastError(), "scratch clear launch"))) return st;
    return q4_gemm_impl(w, nullptr, a, lda, out, ldc, out_dtype, residual, rows, kernel, ptr, kScratchBytes, stream);
}

int splosh_q4_gemm_group(const splosh_q4_weight *weights, int count, const uint16_t *a, int64_t lda,
                         void *const *outs, const int64_t *ldcs, int out_dtype, int64_t rows, int kernel,
                         void *workspace, size_t workspace_bytes, hipStream_t stream) {
    if (!weights || !outs || !ldcs) return fail(SPLOSH_ERR_NULL_POINTER, "null weight, output or ldc list");
    if (count < 1 || count > SPLOSH_MAX_GROUP)
        return fail(SPLOSH_ERR_INVALID_SHAPE, "count must be 1.." + std::to_string(SPLOSH_MAX_GROUP));
    int st;
    int64_t columns = 0;
    bool joined = rows <= 64 && (kernel == SPLOSH_KERNEL_AUTO || kernel == SPLOSH_KERNEL_DEQUANT) && lda % 8 == 0 &&
                  aligned(a, 16);
    for (int i = 0; i < count; ++i) {
        const splosh_q4_weight *w = &weights[i];
        if ((st = check_q4_weight(w, "weight"))) return st;
        if (w->inner != weights[0].inner) return fail(SPLOSH_ERR_INVALID_SHAPE, "grouped weights must share inner");
        if ((st = check_io(a, lda, outs[i], ldcs[i], out_dtype, rows, w->rows, w->inner))) return st;
        joined = joined && w->order == SPLOSH_Q4_TILED128 && aligned(w->packed, 16) &&
                 splosh::mma_fits(rows, w->rows, w->inner, w->row_stride_words, lda);
        columns += w->rows;
    }
    joined = joined && splosh::mma_fits(rows, columns, weights[0].inner, 0, lda) &&
             columns * (weights[0].inner / kGroupSize) * 32 < ((int64_t)1 << 32) - 256;
    if (!joined) {
        for (int i = 0; i < count; ++i)
            if ((st = q4_gemm_impl(&weights[i], nullptr, a, lda, outs[i], ldcs[i], out_dtype, nullptr, rows, kernel,
                                   workspace, workspace_bytes, stream)))
                return st;
        return ok();
    }
    const splosh::MmaPlan plan =
        splosh::plan_mma(rows, columns, weights[0].inner / kGroupSize, false, workspace ? workspace_bytes : 0);
    return hip_status(splosh::launch_q4_mma_group(plan, weights, count, outs, ldcs, a, lda, out_dtype, rows, workspace,
                                                  stream),
                      "q4 grouped mma launch");
}

int splosh_q4_mlp_in(const splosh_q4_weight *gate, const splosh_q4_weight *up, const uint16_t *a, int64_t lda,
                     void *out, int64_t ldc, int out_dtype, int64_t rows, int kernel, void *workspace,
                     size_t workspace_bytes, hipStream_t stream) {
    if (!up) return fail(SPLOSH_ERR_NULL_POINTER, "null up weight");
    return q4_gemm_impl(gate, up, a, lda, out, ldc, out_dtype, nullptr, rows, kernel, workspace, workspace_bytes,
                        stream);
}

int splosh_q4_dequant(const splosh_q4_weight *w, float *out, hipStream_t stream) {
    int st = check_q4_weight(w, "weight");
    if (st) return st;
    if (!out) return fail(SPLOSH_ERR_NULL_POINTER, "null output");
    return hip_status(splosh::launch_q4_dequant(*w, out, stream), "q4 dequant launch");
}

int splosh_q4_embed(const splosh_q4_weight *w, const uint32_t *tokens, int64_t count, void *out, int64_t ldo,
                    int out_dtype, hipStream_t stream) {
    int st = check_q4_weight(w, "embedding");
    if (st) return st;
    if (!tokens || !out) return fail(SPLOSH_ERR_NULL_POINTER, "null tokens or output");
    if (count <= 0) return fail(SPLOSH_ERR_INVALID_SHAPE, "count must be positive");
    if (ldo < w->inner) return fail(SPLOSH_ERR_INVALID_ROW_STRIDE, "ldo is shorter than inner");
    if (out_dtype != SPLOSH_F32 && out_dtype != SPLOSH_BF16) return fail(SPLOSH_ERR_UNSUPPORTED, "unknown out_dtype");
    if (mul_overflows(count, ldo) || count * ((w->inner + 7) / 8) >= ((int64_t)1 << 40))
        return fail(SPLOSH_ERR_ARITHMETIC_OVERFLOW, "size overflows");
    return hip_status(splosh::launch_q4_embed(*w, tokens, count, out, ldo, out_dtype, stream), "q4 embed launch");
}

static int tile_common(const void *src, void *dst, int64_t rows, int64_t groups, int64_t element_bytes, bool inverse,
                       hipStream_t stream) {
    if (!src || !dst) return fail(SPLOSH_ERR_NULL_POINTER, "null buffer");
    if (rows <= 0 || groups <= 0 || element_bytes <= 0 || rows % 128 != 0 || element_bytes % 2 != 0)
        return fail(SPLOSH_ERR_INVALID_SHAPE, "tile needs rows % 128 == 0 and even element bytes");
    if (mul_overflows(rows, groups) || mul_overflows(rows * groups, element_bytes))
        return fail(SPLOSH_ERR_ARITHMETIC_OVERFLOW, "size overflows");
    return hip_status(splosh::launch_tile128(src, dst, rows, groups, element_bytes, inverse, stream), "tile launch");
}

int splosh_tile128(const void *src, void *dst, int64_t rows, int64_t groups, int64_t element_bytes, hipStream_t stream) {
    return tile_common(src, dst, rows, groups, element_bytes, false, stream);
}

int splosh_untile128(const void *src, void *dst, int64_t rows, int64_t groups, int64_t element_bytes,
                     hipStream_t stream) {
    return tile_common(src, dst, rows, groups, element_bytes, true, stream);
}

// The value-head order of a head-ordered weight's inner columns (engine_gguf.metal:55-72): 128
// columns a head, file head h read from engine head vph (h mod kh) + h / kh. key_heads = 0: none.
struct HeadOrder {
    int hs = -1, vph = 0;
    bool on() const { return hs >= 0; }
};
static int head_order(int key_heads, int64_t inner, HeadOrder *out) {
    *out = HeadOrder{};
    if (key_heads == 0) return ok();
    if (key_heads < 0 || (key_heads & (key_heads - 1)) != 0)
        return fail(SPLOSH_ERR_INVALID_SHAPE, "key_heads must be a power of two");
    if (inner % 128 != 0 || (inner / 128) % key_heads != 0)
        return fail(SPLOSH_ERR_INVALID_SHAPE, "inner must be whole 128-column value heads, a multiple of key_heads of them");
    int hs = 0;
    while ((1 << hs) < key_heads) ++hs;
    out->hs = hs;
    out->vph = (int)(inner / 128 / key_heads);
    return ok();
}

// A head-ordered call on a kernel that reads the activations in place: the permuted copy goes to
// the end of the workspace (256-byte aligned), and the kernel gets the rest.
static size_t head_copy_bytes(int64_t m, int64_t inner) { return ((size_t)m * inner * 2 + 255) / 256 * 256; }
static int head_copy(const HeadOrder &ho, const uint16_t **a, int64_t *lda, int64_t m, int64_t inner, void *workspace,
                     size_t *workspace_bytes, hipStream_t stream) {
    const size_t need = head_copy_bytes(m, inner);
    if (!workspace || *workspace_bytes < need)
        return fail(SPLOSH_ERR_WORKSPACE_TOO_SMALL,
                    "a head-ordered weight at this row count needs a workspace of splosh_heads_workspace_bytes()");
    const size_t rest = (*workspace_bytes - need) / 256 * 256;
    uint16_t *dst = (uint16_t *)((char *)workspace + rest);
    int st = hip_status(splosh::launch_head_gather(*a, *lda, m, inner, ho.hs, ho.vph, dst, stream), "head gather launch");
    if (st) return st;
    *a = dst;
    *lda = inner;
    *workspace_bytes = rest;
    return ok();
}

static int gguf_gemm(const splosh_q5k_weight *w_in, bool fifth, const uint16_t *a, int64_t lda, void *out, int64_t ldc,
                     int out_dtype, const void *residual, int64_t rows, int kernel, void *workspace,
                     size_t workspace_bytes, hipStream_t stream, int key_heads = 0) {
    int st = check_q5k_weight(w_in, fifth);
    if (st) return st;
    HeadOrder ho;
    if ((st = head_order(key_heads, w_in->inner, &ho))) return st;
    splosh_q5k_weight wv = *w_in;
    if (!fifth) wv.plane1 = nullptr;  // the kernels read no fifth bits
    const splosh_q5k_weight *w = &wv;
    if ((st = check_io(a, lda, out, ldc, out_dtype, rows, w->rows, w->inner))) return st;
    const bool planes_ok = aligned(w->plane0, 16) && (!fifth || aligned(w->plane1, 4)) && aligned(w->meta, 16);
    // 65..128 rows under AUTO: two calls of at most 64 rows, as for q4 (K17408 -> N5120, against the
    // prefill kernel: M=96 66 -> 54 us, M=128 69 -> 59).
    if (kernel == SPLOSH_KERNEL_AUTO && rows > 64 && rows <= 128 && planes_ok && lda % 8 == 0 && aligned(a, 16) &&
        splosh::q5k_mma_fits(64, w->rows, w->inner, lda)) {
        const char *res = (const char *)residual;
        const size_t esize = out_dtype == SPLOSH_F32 ? 4 : 2;
        if ((st = gguf_gemm(w_in, fifth, a, lda, out, ldc, out_dtype, residual, 64, kernel, workspace,
                            workspace_bytes, stream, key_heads)))
            return st;
        return gguf_gemm(w_in, fifth, a + 64 * lda, lda, (char *)out + 64 * ldc * esize, ldc, out_dtype,
                             res ? res + 64 * ldc * esize : nullptr, rows - 64, kernel, workspace, workspace_bytes,
                             stream, key_heads);
    }
    if (kernel == SPLOSH_KERNEL_AUTO && planes_ok && lda % 4 == 0 && aligned(a, 16) &&
        splosh::q5k_decode_fits(rows, w->rows, w->inner))
        return hip_status(splosh::launch_q5k_decode(*w, a, out, out_dtype, residual, workspace,
                                                    workspace ? workspace_bytes : 0, stream, ho.hs, ho.vph),
                          "q5k decode launch");
    // Every other kernel reads the activations in place: a head-ordered call gives it a permuted
    // copy (dense rows of `inner`, 256-byte aligned, at the end of the workspace).
    if (ho.on()) {
        if (lda % 8 != 0 || !aligned(a, 16))
            return fail(SPLOSH_ERR_UNSUPPORTED, "head-ordered GEMM needs lda % 8 == 0 and 16-byte aligned activations");
        if ((st = head_copy(ho, &a, &lda, rows, w->inner, workspace, &workspace_bytes, stream))) return st;
        if (workspace_bytes == 0) workspace = nullptr;
    }
    const bool eligible = lda % 4 == 0 && aligned(a, 8) && planes_ok;
    const bool mma_ok = eligible && lda % 8 == 0 && aligned(a, 16) && splosh::q5k_mma_fits(rows, w->rows, w->inner, lda);
    const bool tile_ok = eligible && lda % 8 == 0 && aligned(a, 16) && splosh::gguf_tile_fits(rows, w->rows, w->inner, lda);
    const bool prefill_ok = eligible && lda % 8 == 0 && aligned(a, 16) && aligned(out, 16) &&
                            (!residual || aligned(residual, 16)) &&
                            splosh::q5k_prefill_fits(rows, w->rows, w->inner, lda, ldc);
    int choice = kernel;
    if (kernel == SPLOSH_KERNEL_AUTO) {
        if (!eligible) choice = SPLOSH_KERNEL_SCALAR;
        else if (mma_ok) choice = SPLOSH_KERNEL_DEQUANT;
        // Above 64 rows the 256 x 256 prefill kernel (K17408 -> N5120: 75 us at 128 rows against the
        // tile kernel's 86, 381 against 627 at 2048).
        else if (prefill_ok) choice = SPLOSH_KERNEL_PREFILL;
        else if (tile_ok) choice = SPLOSH_KERNEL_TILE;
        else choice = SPLOSH_KERNEL_STREAM;
    }
    switch (choice) {
        case SPLOSH_KERNEL_PREFILL: {
            if (!prefill_ok)
                return fail(SPLOSH_ERR_UNSUPPORTED,
                            "prefill kernel needs K % 256 == 0, N % 128 == 0, lda % 8 == 0, ldc % 4 == 0 and 16-byte "
                            "aligned operands");
            const splosh::PrefillPlan plan =
                splosh::plan_prefill(rows, w->rows, w->inner / kGroupSize, workspace ? workspace_bytes : 0);
            return hip_status(splosh::launch_q5k_prefill(plan, *w, fifth, a, lda, out, ldc, out_dtype, residual, rows,
                                                         workspace, stream),
                              "q5k prefill launch");
        }
        case SPLOSH_KERNEL_TILE:
            if (!tile_ok) return fail(SPLOSH_ERR_UNSUPPORTED, "tile kernel needs lda % 8 == 0 and aligned operands");
            return hip_status(splosh::launch_gguf_tile(fifth ? 13 : 12, w->plane0, w->plane1, w->meta, w->rows,
                                                       w->inner, a, lda, out, ldc, out_dtype, residual, rows,
                                                       workspace, workspace_bytes, stream),
                              "gguf tile launch");
        case SPLOSH_KERNEL_STREAM: {
            if (!eligible) return fail(SPLOSH_ERR_UNSUPPORTED, "stream kernel needs lda % 4 == 0 and aligned planes");
            const splosh::StreamPlan plan = splosh::plan_stream(rows, w->rows, w->inner / 256, false, 2);
            if (plan.row_chunks > 65535) return fail(SPLOSH_ERR_UNSUPPORTED, "too many rows for one launch");
            return hip_status(splosh::launch_q5k_stream(plan, *w, a, lda, out, ldc, out_dtype, residual, rows, stream),
                              "q5k stream launch");
        }
        case SPLOSH_KERNEL_DEQUANT: {
            if (!mma_ok) return fail(SPLOSH_ERR_UNSUPPORTED, "dequant kernel needs rows <= 64 and aligned operands");
            const splosh::MmaPlan plan =
                splosh::plan_mma(rows, w->rows, w->inner / 256, false, workspace ? workspace_bytes : 0, 256);
            return hip_status(splosh::launch_q5k_mma(plan, *w, a, lda, out, ldc, out_dtype, residual, rows, workspace,
                                                     stream),
                              "q5k dequant launch");
        }
        case SPLOSH_KERNEL_SCALAR:
            if (rows > 65535) return fail(SPLOSH_ERR_UNSUPPORTED, "scalar kernel takes at most 65535 rows");
            return hip_status(splosh::launch_q5k_gemm_scalar(*w, a, lda, out, ldc, out_dtype, residual, rows, stream),
                              "q5k scalar launch");
        default:
            return fail(SPLOSH_ERR_UNSUPPORTED, "kernel not available for Q5_K in this build");
    }
}

static int gguf_dequant(const splosh_q5k_weight *w, bool fifth, float *out, hipStream_t stream) {
    int st = check_q5k_weight(w, fifth);
    if (st) return st;
    if (!out) return fail(SPLOSH_ERR_NULL_POINTER, "null output");
    splosh_q5k_weight wv = *w;
    if (!fifth) wv.plane1 = nullptr;
    return hip_status(splosh::launch_q5k_dequant(wv, out, stream), "gguf dequant launch");
}

int splosh_q5k_gemm(const splosh_q5k_weight *w, const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                    const void *residual, int64_t rows, int kernel, void *workspace, size_t workspace_bytes,
                    hipStream_t stream) {
    return gguf_gemm(w, true, a, lda, out, ldc, out_dtype, residual, rows, kernel, workspace, workspace_bytes, stream);
}

int splosh_q4k_gemm(const splosh_q5k_weight *w, const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                    const void *residual, int64_t rows, int kernel, void *workspace, size_t workspace_bytes,
                    hipStream_t stream) {
    return gguf_gemm(w, false, a, lda, out, ldc, out_dtype, residual, rows, kernel, workspace, workspace_bytes, stream);
}

// The `heads` kernels of engine_gguf.metal:336-338 (Engine.swift:765-779, ggufHeadOrder).
int splosh_q5k_gemm_heads(const splosh_q5k_weight *w, int key_heads, const uint16_t *a, int64_t lda, void *out,
                          int64_t ldc, int out_dtype, const void *residual, int64_t rows, int kernel, void *workspace,
                          size_t workspace_bytes, hipStream_t stream) {
    if (key_heads <= 0) return fail(SPLOSH_ERR_INVALID_SHAPE, "key_heads must be positive");
    return gguf_gemm(w, true, a, lda, out, ldc, out_dtype, residual, rows, kernel, workspace, workspace_bytes, stream,
                     key_heads);
}

int splosh_q4k_gemm_heads(const splosh_q5k_weight *w, int key_heads, const uint16_t *a, int64_t lda, void *out,
                          int64_t ldc, int out_dtype, const void *residual, int64_t rows, int kernel, void *workspace,
                          size_t workspace_bytes, hipStream_t stream) {
    if (key_heads <= 0) return fail(SPLOSH_ERR_INVALID_SHAPE, "key_heads must be positive");
    return gguf_gemm(w, false, a, lda, out, ldc, out_dtype, residual, rows, kernel, workspace, workspace_bytes, stream,
                     key_heads);
}

size_t splosh_heads_workspace_bytes(int64_t rows, int64_t columns, int64_t inner) {
    if (rows <= 0 || columns <= 0 || inner <= 0) return 0;
    return splosh_workspace_bytes(rows, columns, inner) + 256 + head_copy_bytes(rows, inner);
}

int splosh_q5k_dequant(const splosh_q5k_weight *w, float *out, hipStream_t stream) {
    return gguf_dequant(w, true, out, stream);
}

int splosh_q4k_dequant(const splosh_q5k_weight *w, float *out, hipStream_t stream) {
    return gguf_dequant(w, false, out, stream);
}

// Shape and geometry checks shared by the native-block GGUF entry points.
static int check_gguf_native(int type, const uint8_t *native, int64_t rows, int64_t inner) {
    int elems = 0, bytes = 0;
    if ((type & ~(0xFF | SPLOSH_GGUF_ROWS32)) != 0 || !splosh::gguf_native_block(type, &elems, &bytes))
        return fail(SPLOSH_ERR_UNSUPPORTED, "ggml type not supported in native blocks (Q8_0, Q3_K, Q6_K, IQ4_NL, IQ3_S, IQ4_XS)");
    const bool rows32 = (type & SPLOSH_GGUF_ROWS32) != 0;
    if (rows32 && (inner <= 0 || inner % 256 != 0))
        return fail(SPLOSH_ERR_LAYOUT_MISMATCH, "the ROWS32 layout needs inner % 256 == 0");
    if (!native) return fail(SPLOSH_ERR_NULL_POINTER, "null weight");
    // The kernels read the blocks through dword-aligned windows relative to this base (GGUF tensor
    // data is 32-byte aligned in the file).
    if (!aligned(native, 4)) return fail(SPLOSH_ERR_LAYOUT_MISMATCH, "native weight must be 4-byte aligned");
    if (rows <= 0 || inner <= 0) return fail(SPLOSH_ERR_INVALID_SHAPE, "rows and inner must be positive");
    if (inner % elems != 0) return fail(SPLOSH_ERR_LAYOUT_MISMATCH, "inner is not a whole number of native blocks");
    const int64_t stored = rows32 ? (rows + 31) / 32 * 32 : rows;  // ROWS32 pads to whole groups of 32 rows
    if (mul_overflows(stored, inner / elems * bytes) || stored * (inner / elems * bytes) >= ((int64_t)1 << 32))
        return fail(SPLOSH_ERR_ARITHMETIC_OVERFLOW, "weight larger than 4 GiB");
    return ok();
}

constexpr int64_t kGgufPrefillRows = 256;  // measured: the tile kernel is as fast or faster up to 128 rows

static int gguf_native_gemm(int gguf_type, const uint8_t *native, int64_t rows, int64_t inner, const uint16_t *a,
                            int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual, int64_t m,
                            void *workspace, size_t workspace_bytes, hipStream_t stream, int key_heads) {
    int st = check_gguf_native(gguf_type, native, rows, inner);
    if (st) return st;
    if ((st = check_io(a, lda, out, ldc, out_dtype, m, rows, inner))) return st;
    if (lda % 8 != 0 || !aligned(a, 16))
        return fail(SPLOSH_ERR_UNSUPPORTED, "GGUF native kernel needs lda % 8 == 0 and 16-byte aligned activations");
    HeadOrder ho;
    if ((st = head_order(key_heads, inner, &ho))) return st;
    // From kGgufPrefillRows rows the 256 x 256 prefill kernel (each weight group decoded once per
    // 256 rows). Up to 64 rows the stream-K MFMA kernel (each weight group decoded once), above
    // the format's streaming limit; up to it one pass of the streaming kernel. Measured at K17408
    // -> N5120 with a workspace (us): the MFMA kernel is flat up to 32 rows (Q8_0 33, Q6_K 44, Q3_K
    // 47, IQ3_S 42, IQ4_NL 27, IQ4_XS 30); the streaming kernel at four rows Q8_0 31, Q6_K 35, Q3_K
    // 32, IQ3_S 31, IQ4_NL 29, IQ4_XS 29, at five Q6_K 45, Q3_K 43, IQ3_S 43, at six Q3_K 47, at
    // three IQ4_NL 26. Where the MFMA kernel does not fit (K % 256 != 0), the streaming kernel
    // serves up to eight rows and the LDS-tiled kernel above. (A development override of the
    // prefill threshold, read once.)
    static const int64_t prefill_rows = [] {
        const char *e = getenv("SPLOSH_GGUF_PREFILL_ROWS");
        return e ? (int64_t)atoll(e) : kGgufPrefillRows;
    }();
    const bool prefill = m >= prefill_rows && aligned(out, 16) && (!residual || aligned(residual, 16)) &&
                         splosh::gguf_prefill_fits(gguf_type, m, rows, inner, lda, ldc);
    const int base_type = gguf_type & 0xFF;
    const int64_t stream_max = base_type == 11 ? 6 : base_type == 20 ? 3 : 4;
    // 65..128 rows: two calls of at most 64 rows, as for q4. K17408 -> N5120, against the tiled
    // kernel: M=96 Q8_0 80 -> 77 us (ROWS32 79 -> 66), Q6_K 100 -> 90, IQ3_S 105 -> 89, IQ4_NL 81 ->
    // 63, IQ4_XS 81 -> 70; Q3_K, whose MFMA path is the slowest, 83 -> 96, keeps the tiled kernel.
    if (base_type != 11 && m > 64 && m <= 128 && splosh::gguf_mma_fits(gguf_type, 64, rows, inner, lda)) {
        const char *res = (const char *)residual;
        const size_t esize = out_dtype == SPLOSH_F32 ? 4 : 2;
        if ((st = gguf_native_gemm(gguf_type, native, rows, inner, a, lda, out, ldc, out_dtype, residual, 64,
                                   workspace, workspace_bytes, stream, key_heads)))
            return st;
        return gguf_native_gemm(gguf_type, native, rows, inner, a + 64 * lda, lda, (char *)out + 64 * ldc * esize,
                                ldc, out_dtype, res ? res + 64 * ldc * esize : nullptr, m - 64, workspace,
                                workspace_bytes, stream, key_heads);
    }
    const bool mma = !prefill && m > stream_max && splosh::gguf_mma_fits(gguf_type, m, rows, inner, lda);
    const bool tile = !prefill && !mma && m > 8 && splosh::gguf_tile_fits(m, rows, inner, lda);
    // The streaming kernels read the activations through head_group(); the other kernels get a
    // permuted copy.
    if (ho.on() && (prefill || mma || tile)) {
        if ((st = head_copy(ho, &a, &lda, m, inner, workspace, &workspace_bytes, stream))) return st;
        if (workspace_bytes == 0) workspace = nullptr;
    }
    if (prefill) {
        const splosh::PrefillPlan plan = splosh::plan_prefill(m, rows, inner / kGroupSize, workspace ? workspace_bytes : 0);
        return hip_status(splosh::launch_gguf_prefill(plan, gguf_type, native, rows, inner, a, lda, out, ldc, out_dtype,
                                                      residual, m, workspace, stream),
                          "gguf prefill launch");
    }
    if (mma) {
        const splosh::MmaPlan plan =
            splosh::plan_mma(m, rows, inner / 256, false, workspace ? workspace_bytes : 0, 256);
        return hip_status(splosh::launch_gguf_mma(plan, gguf_type, native, rows, inner, a, lda, out, ldc, out_dtype,
                                                  residual, m, workspace, stream),
                          "gguf mma launch");
    }
    if (tile)
        return hip_status(splosh::launch_gguf_tile(gguf_type, native, nullptr, nullptr, rows, inner, a, lda, out, ldc,
                                                   out_dtype, residual, m, workspace, workspace_bytes, stream),
                          "gguf tile launch");
    if (m > ((int64_t)65535 * 4)) return fail(SPLOSH_ERR_UNSUPPORTED, "too many activation rows for one launch");
    return hip_status(splosh::launch_gguf_gemv(gguf_type, native, rows, inner, a, lda, out, ldc, out_dtype, residual,
                                               m, stream, ho.hs, ho.vph),
                      "gguf native gemm launch");
}

size_t splosh_gguf_rows32_bytes(int gguf_type, int64_t rows, int64_t inner) {
    int elems = 0, bytes = 0;
    if ((gguf_type & ~0xFF) != 0 || !splosh::gguf_native_block(gguf_type, &elems, &bytes) || rows <= 0 ||
        inner <= 0 || inner % 256 != 0)
        return 0;
    return (size_t)((rows + 31) / 32 * 32) * (size_t)(inner / elems * bytes);
}

int splosh_gguf_repack_rows32(int gguf_type, const uint8_t *native, int64_t rows, int64_t inner, uint8_t *out,
                              hipStream_t stream) {
    if (gguf_type & SPLOSH_GGUF_ROWS32) return fail(SPLOSH_ERR_LAYOUT_MISMATCH, "the source must be in the file's order");
    int st = check_gguf_native(gguf_type | SPLOSH_GGUF_ROWS32, native, rows, inner);
    if (st) return st;
    if (!out) return fail(SPLOSH_ERR_NULL_POINTER, "null output");
    if (!aligned(out, 4)) return fail(SPLOSH_ERR_LAYOUT_MISMATCH, "output must be 4-byte aligned");
    return hip_status(splosh::launch_gguf_repack_rows32(gguf_type, native, rows, inner, out, stream),
                      "gguf rows32 repack launch");
}

int splosh_gguf_gemm(int gguf_type, const uint8_t *native, int64_t rows, int64_t inner, const uint16_t *a,
                     int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual, int64_t m,
                     void *workspace, size_t workspace_bytes, hipStream_t stream) {
    return gguf_native_gemm(gguf_type, native, rows, inner, a, lda, out, ldc, out_dtype, residual, m, workspace,
                            workspace_bytes, stream, 0);
}

int splosh_gguf_gemm_heads(int gguf_type, const uint8_t *native, int64_t rows, int64_t inner, int key_heads,
                           const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual,
                           int64_t m, void *workspace, size_t workspace_bytes, hipStream_t stream) {
    if (key_heads <= 0) return fail(SPLOSH_ERR_INVALID_SHAPE, "key_heads must be positive");
    return gguf_native_gemm(gguf_type, native, rows, inner, a, lda, out, ldc, out_dtype, residual, m, workspace,
                            workspace_bytes, stream, key_heads);
}

int splosh_gguf_dequant(int gguf_type, const uint8_t *native, int64_t rows, int64_t inner, float *out,
                        hipStream_t stream) {
    int st = check_gguf_native(gguf_type, native, rows, inner);
    if (st) return st;
    if (!out || !aligned(out, 16)) return fail(SPLOSH_ERR_NULL_POINTER, "null or unaligned output");
    return hip_status(splosh::launch_gguf_dequant(gguf_type, native, rows, inner, out, stream),
                      "gguf native dequant launch");
}

// Checks shared by the embedding lookups: ids, output and its row stride.
static int check_embed_io(const uint32_t *tokens, int64_t count, const void *out, int64_t ldo, int64_t inner,
                          int out_dtype) {
    if (!tokens || !out) return fail(SPLOSH_ERR_NULL_POINTER, "null tokens or output");
    if (count <= 0) return fail(SPLOSH_ERR_INVALID_SHAPE, "count must be positive");
    if (ldo < inner) return fail(SPLOSH_ERR_INVALID_ROW_STRIDE, "ldo is shorter than inner");
    if (out_dtype != SPLOSH_F32 && out_dtype != SPLOSH_BF16) return fail(SPLOSH_ERR_UNSUPPORTED, "unknown out_dtype");
    if (mul_overflows(count, ldo) || count * (inner / 32) >= ((int64_t)1 << 40))
        return fail(SPLOSH_ERR_ARITHMETIC_OVERFLOW, "size overflows");
    return SPLOSH_OK;
}

static int gguf_embed_planes(const splosh_q5k_weight *w, bool fifth, const uint32_t *tokens, int64_t count, void *out,
                             int64_t ldo, int out_dtype, hipStream_t stream) {
    int st = check_q5k_weight(w, fifth);
    if (st) return st;
    if ((st = check_embed_io(tokens, count, out, ldo, w->inner, out_dtype))) return st;
    splosh_q5k_weight wv = *w;
    if (!fifth) wv.plane1 = nullptr;
    return hip_status(splosh::launch_q5k_embed(wv, tokens, count, out, ldo, out_dtype, stream), "gguf embed launch");
}

int splosh_q5k_embed(const splosh_q5k_weight *w, const uint32_t *tokens, int64_t count, void *out, int64_t ldo,
                     int out_dtype, hipStream_t stream) {
    return gguf_embed_planes(w, true, tokens, count, out, ldo, out_dtype, stream);
}

int splosh_q4k_embed(const splosh_q5k_weight *w, const uint32_t *tokens, int64_t count, void *out, int64_t ldo,
                     int out_dtype, hipStream_t stream) {
    return gguf_embed_planes(w, false, tokens, count, out, ldo, out_dtype, stream);
}

int splosh_gguf_embed(int gguf_type, const uint8_t *native, int64_t rows, int64_t inner, const uint32_t *tokens,
                      int64_t count, void *out, int64_t ldo, int out_dtype, hipStream_t stream) {
    int st = check_gguf_native(gguf_type, native, rows, inner);
    if (st) return st;
    if ((st = check_embed_io(tokens, count, out, ldo, inner, out_dtype))) return st;
    return hip_status(splosh::launch_gguf_embed(gguf_type, native, rows, inner, tokens, count, out, ldo, out_dtype,
                                                stream),
                      "gguf native embed launch");
}

// The repack kernels move native blocks in dwords and plane records in 16-byte pieces.
static int check_plane_alignment(const uint8_t *native, const uint8_t *plane0, const uint8_t *plane1,
                                 const uint8_t *meta) {
    if (!aligned(native, 4) || !aligned(plane0, 16) || (plane1 && !aligned(plane1, 4)) || !aligned(meta, 16))
        return fail(SPLOSH_ERR_LAYOUT_MISMATCH, "native blocks need 4-byte, plane0 and meta 16-byte, plane1 4-byte alignment");
    return ok();
}

int splosh_q5k_repack(const uint8_t *native, int64_t rows, int64_t inner, uint8_t *plane0, uint8_t *plane1,
                      uint8_t *meta, hipStream_t stream) {
    if (!native || !plane0 || !plane1 || !meta) return fail(SPLOSH_ERR_NULL_POINTER, "null buffer");
    if (rows <= 0 || inner <= 0 || rows % 128 != 0 || inner % 256 != 0)
        return fail(SPLOSH_ERR_LAYOUT_MISMATCH, "Q5_K planes need rows % 128 == 0 and inner % 256 == 0");
    if (int st = check_plane_alignment(native, plane0, plane1, meta)) return st;
    return hip_status(splosh::launch_q5k_repack(native, rows, inner, plane0, plane1, meta, false, stream),
                      "q5k repack launch");
}

int splosh_q4k_repack(const uint8_t *native, int64_t rows, int64_t inner, uint8_t *plane0, uint8_t *meta,
                      hipStream_t stream) {
    if (!native || !plane0 || !meta) return fail(SPLOSH_ERR_NULL_POINTER, "null buffer");
    if (rows <= 0 || inner <= 0 || rows % 128 != 0 || inner % 256 != 0)
        return fail(SPLOSH_ERR_LAYOUT_MISMATCH, "Q4_K planes need rows % 128 == 0 and inner % 256 == 0");
    if (int st = check_plane_alignment(native, plane0, nullptr, meta)) return st;
    return hip_status(splosh::launch_q5k_repack(native, rows, inner, plane0, nullptr, meta, false, stream, false),
                      "q4k repack launch");
}

int splosh_q4k_unpack(const uint8_t *plane0, const uint8_t *meta, int64_t rows, int64_t inner, uint8_t *native,
                      hipStream_t stream) {
    if (!native || !plane0 || !meta) return fail(SPLOSH_ERR_NULL_POINTER, "null buffer");
    if (rows <= 0 || inner <= 0 || rows % 128 != 0 || inner % 256 != 0)
        return fail(SPLOSH_ERR_LAYOUT_MISMATCH, "Q4_K planes need rows % 128 == 0 and inner % 256 == 0");
    if (int st = check_plane_alignment(native, plane0, nullptr, meta)) return st;
    return hip_status(splosh::launch_q5k_repack(native, rows, inner, const_cast<uint8_t *>(plane0), nullptr,
                                                const_cast<uint8_t *>(meta), true, stream, false),
                      "q4k unpack launch");
}

int splosh_q5k_unpack(const uint8_t *plane0, const uint8_t *plane1, const uint8_t *meta, int64_t rows, int64_t inner,
                      uint8_t *native, hipStream_t stream) {
    if (!native || !plane0 || !plane1 || !meta) return fail(SPLOSH_ERR_NULL_POINTER, "null buffer");
    if (rows <= 0 || inner <= 0 || rows % 128 != 0 || inner % 256 != 0)
        return fail(SPLOSH_ERR_LAYOUT_MISMATCH, "Q5_K planes need rows % 128 == 0 and inner % 256 == 0");
    if (int st = check_plane_alignment(native, plane0, plane1, meta)) return st;
    return hip_status(splosh::launch_q5k_repack(native, rows, inner, const_cast<uint8_t *>(plane0),
                                                const_cast<uint8_t *>(plane1), const_cast<uint8_t *>(meta), true,
                                                stream),
                      "q5k unpack launch");
}

}  // extern "C"

// ---- operand producers ---------------------------------------------------------------------

namespace {

int check_operand_io(const void *in, int64_t ld_in, int64_t rows, int64_t dim, const void *out, int64_t ld_out,
                     const void *sums) {
    if (!in || !out || !sums) return fail(SPLOSH_ERR_NULL_POINTER, "null operand pointer");
    if (rows <= 0 || dim <= 0) return fail(SPLOSH_ERR_INVALID_SHAPE, "rows and dim must be positive");
    if (dim % 64 != 0) return fail(SPLOSH_ERR_INVALID_GROUP_SIZE, "dim must be a multiple of 64");
    if (ld_in < dim || ld_out < dim) return fail(SPLOSH_ERR_INVALID_ROW_STRIDE, "row stride shorter than dim");
    if (ld_in % 4 != 0 || !aligned(in, 16) || ld_out % 4 != 0 || !aligned(out, 8))
        return fail(SPLOSH_ERR_UNSUPPORTED, "operand kernels need 16-byte fp32 rows and 8-byte bf16 rows");
    if (mul_overflows(rows, ld_in) || mul_overflows(rows, ld_out) || rows * (dim / 4) >= ((int64_t)1 << 40))
        return fail(SPLOSH_ERR_ARITHMETIC_OVERFLOW, "size overflows");
    return SPLOSH_OK;
}

}  // namespace

extern "C" {

int splosh_prepare_operand(const float *x, int64_t ldx, int64_t rows, int64_t dim, uint16_t *out, int64_t ld_out,
                           float *sums, hipStream_t stream) {
    int st = check_operand_io(x, ldx, rows, dim, out, ld_out, sums);
    if (st) return st;
    return hip_status(splosh::launch_prepare_operand(x, ldx, rows, dim, out, ld_out, sums, stream), "prepare launch");
}

int splosh_silu_mul_operand(const float *gate, const float *up, int64_t ld, const float *row_inv, int64_t rows,
                            int64_t dim, uint16_t *out, int64_t ld_out, float *sums, hipStream_t stream) {
    int st = check_operand_io(gate, ld, rows, dim, out, ld_out, sums);
    if (st) return st;
    if (!up) return fail(SPLOSH_ERR_NULL_POINTER, "null up pointer");
    if (!aligned(up, 16)) return fail(SPLOSH_ERR_UNSUPPORTED, "up must be 16-byte aligned");
    return hip_status(splosh::launch_silu_mul_operand(gate, up, ld, row_inv, rows, dim, out, ld_out, sums, stream),
                      "silu_mul launch");
}

int splosh_emit_operand(const float *hidden, int64_t ld_hidden, const uint16_t *norm_weight, int64_t rows,
                        int64_t dim, uint16_t *values, int64_t ld_values, float *sums, float *squares,
                        hipStream_t stream) {
    int st = check_operand_io(hidden, ld_hidden, rows, dim, values, ld_values, sums);
    if (st) return st;
    if (!norm_weight || !squares) return fail(SPLOSH_ERR_NULL_POINTER, "null norm weight or squares");
    if (!aligned(norm_weight, 8)) return fail(SPLOSH_ERR_UNSUPPORTED, "norm weight must be 8-byte aligned");
    return hip_status(splosh::launch_emit_operand(hidden, ld_hidden, norm_weight, rows, dim, values, ld_values, sums,
                                                  squares, stream),
                      "emit launch");
}

int splosh_row_inv(const float *squares, int64_t rows, int64_t groups, int64_t dim, float eps, float *inv,
                   hipStream_t stream) {
    if (!squares || !inv) return fail(SPLOSH_ERR_NULL_POINTER, "null squares or inv");
    if (rows <= 0 || groups <= 0 || dim <= 0) return fail(SPLOSH_ERR_INVALID_SHAPE, "rows, groups and dim must be positive");
    if (rows > 0x7fffffff) return fail(SPLOSH_ERR_UNSUPPORTED, "too many rows for one launch");
    return hip_status(splosh::launch_row_inv(squares, rows, groups, dim, eps, inv, stream), "row_inv launch");
}

}  // extern "C"
