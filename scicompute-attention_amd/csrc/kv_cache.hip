// KV cache data movement over the block-major layout [num_blocks][block_size][H_kv][D].
//
// Behaviour follows src/kv_cache/kv_cache_kernels.cu:17-86 of the reference (scatter-append by
// slot with slot < 0 / out-of-pool blocks skipped, block reset to zero, block gather into a
// contiguous buffer). The MI355X versions move whole token rows ([H_kv][D] is contiguous in both
// the staging tensor and a cache slot) with 16-byte vector accesses, one lane per 16 B, so the
// copies run at HBM speed instead of byte-per-thread.

#include <hip/hip_runtime.h>

#include <string>

#include "sca_device.hpp"

namespace sca_hip {
namespace {

constexpr int kThreads = 256;
constexpr int64_t kMaxGrid = 65535;

__global__ void kv_append_kernel(uint4* __restrict__ layer_k, uint4* __restrict__ layer_v,
                                 const uint4* __restrict__ k_new, const uint4* __restrict__ v_new,
                                 const int32_t* __restrict__ slots, int64_t num_tokens,
                                 int64_t row_chunks, int64_t block_size, int64_t num_blocks) {
    const int64_t total = num_tokens * row_chunks;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += stride) {
        const int64_t t = i / row_chunks;
        const int64_t c = i - t * row_chunks;
        const int64_t slot = slots[t];
        if (slot < 0 || slot / block_size >= num_blocks) continue;
        layer_k[slot * row_chunks + c] = k_new[i];
        layer_v[slot * row_chunks + c] = v_new[i];
    }
}

__global__ void kv_reset_kernel(uint4* __restrict__ layer_k, uint4* __restrict__ layer_v,
                                const int32_t* __restrict__ block_ids, int64_t n_ids,
                                int64_t block_chunks, int64_t num_blocks) {
    const int64_t total = n_ids * block_chunks;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    const uint4 zero = make_uint4(0u, 0u, 0u, 0u);
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += stride) {
        const int64_t n = i / block_chunks;
        const int64_t c = i - n * block_chunks;
        const int64_t block = block_ids[n];
        if (block < 0 || block >= num_blocks) continue;
        layer_k[block * block_chunks + c] = zero;
        layer_v[block * block_chunks + c] = zero;
    }
}

__global__ void kv_gather_kernel(const uint4* __restrict__ layer, const int32_t* __restrict__ ids,
                                 int64_t n_ids, uint4* __restrict__ out, int64_t block_chunks,
                                 int64_t num_blocks) {
    const int64_t total = n_ids * block_chunks;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += stride) {
        const int64_t n = i / block_chunks;
        const int64_t c = i - n * block_chunks;
        const int64_t block = ids[n];
        out[i] = (block < 0 || block >= num_blocks) ? make_uint4(0u, 0u, 0u, 0u)
                                                    : layer[block * block_chunks + c];
    }
}

// dst[pairs[2i]] = pairs[2i+1]; indices outside [0, dst_len) are skipped.
__global__ void i32_scatter_kernel(int32_t* __restrict__ dst, int64_t dst_len,
                                   const int2* __restrict__ pairs, int64_t num_pairs) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < num_pairs;
         i += stride) {
        const int2 pr = pairs[i];
        if (pr.x >= 0 && pr.x < dst_len) dst[pr.x] = pr.y;
    }
}

unsigned GridFor(int64_t total) {
    int64_t blocks = (total + kThreads - 1) / kThreads;
    if (blocks < 1) blocks = 1;
    if (blocks > kMaxGrid) blocks = kMaxGrid;
    return static_cast<unsigned>(blocks);
}

int CheckShape(const sca_kv_shape* shape, int64_t elem_bytes, const char* what,
               int64_t* row_bytes) {
    if (shape == nullptr) return SetError(SCA_E_SHAPE_MISMATCH, std::string(what) + ": null shape");
    if (shape->num_blocks <= 0 || shape->block_size <= 0 || shape->num_kv_heads <= 0 ||
        shape->head_dim <= 0) {
        return SetError(SCA_E_SHAPE_MISMATCH, std::string(what) + ": non-positive KV geometry");
    }
    if (elem_bytes != 2 && elem_bytes != 4) {
        return SetError(SCA_E_UNSUPPORTED_DTYPE,
                        std::string(what) + ": elem_bytes=" + std::to_string(elem_bytes));
    }
    *row_bytes = shape->num_kv_heads * shape->head_dim * elem_bytes;
    if (*row_bytes % 16 != 0) {
        return SetError(SCA_E_UNSUPPORTED_HEAD_DIM,
                        std::string(what) + ": token row of " + std::to_string(*row_bytes) +
                            " B is not a multiple of 16 B");
    }
    return 0;
}

bool Aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace sca_hip

using sca_hip::SetError;

extern "C" {

int sca_hip_kv_append(void* layer_k, void* layer_v, const void* k_new, const void* v_new,
                      const int32_t* slot_mapping, int64_t num_tokens, const sca_kv_shape* shape,
                      int64_t elem_bytes, void* stream) {
    int64_t row_bytes = 0;
    int rc = sca_hip::CheckShape(shape, elem_bytes, "kv_append", &row_bytes);
    if (rc != 0) return rc;
    if (num_tokens <= 0) return 0;
    if (layer_k == nullptr || layer_v == nullptr || k_new == nullptr || v_new == nullptr ||
        slot_mapping == nullptr) {
        return SetError(SCA_E_SHAPE_MISMATCH, "kv_append: null pointer");
    }
    if (!sca_hip::Aligned16(layer_k) || !sca_hip::Aligned16(layer_v) ||
        !sca_hip::Aligned16(k_new) || !sca_hip::Aligned16(v_new)) {
        return SetError(SCA_E_LAYOUT_MISMATCH, "kv_append: buffers must be 16 B aligned");
    }
    const int64_t row_chunks = row_bytes / 16;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(sca_hip::kv_append_kernel, dim3(sca_hip::GridFor(num_tokens * row_chunks)),
                       dim3(sca_hip::kThreads), 0, s, static_cast<uint4*>(layer_k),
                       static_cast<uint4*>(layer_v), static_cast<const uint4*>(k_new),
                       static_cast<const uint4*>(v_new), slot_mapping, num_tokens, row_chunks,
                       shape->block_size, shape->num_blocks);
    return sca_hip::CheckLaunch("kv_append_kernel", s);
}

int sca_hip_kv_reset_blocks(void* layer_k, void* layer_v, const int32_t* block_ids,
                            int64_t num_block_ids, const sca_kv_shape* shape, int64_t elem_bytes,
                            void* stream) {
    int64_t row_bytes = 0;
    int rc = sca_hip::CheckShape(shape, elem_bytes, "kv_reset", &row_bytes);
    if (rc != 0) return rc;
    if (num_block_ids <= 0) return 0;
    if (layer_k == nullptr || layer_v == nullptr || block_ids == nullptr) {
        return SetError(SCA_E_SHAPE_MISMATCH, "kv_reset: null pointer");
    }
    if (!sca_hip::Aligned16(layer_k) || !sca_hip::Aligned16(layer_v)) {
        return SetError(SCA_E_LAYOUT_MISMATCH, "kv_reset: buffers must be 16 B aligned");
    }
    const int64_t block_chunks = row_bytes * shape->block_size / 16;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(sca_hip::kv_reset_kernel,
                       dim3(sca_hip::GridFor(num_block_ids * block_chunks)),
                       dim3(sca_hip::kThreads), 0, s, static_cast<uint4*>(layer_k),
                       static_cast<uint4*>(layer_v), block_ids, num_block_ids, block_chunks,
                       shape->num_blocks);
    return sca_hip::CheckLaunch("kv_reset_kernel", s);
}

int sca_hip_kv_gather(const void* layer, const int32_t* block_ids, int64_t num_block_ids,
                      void* out, const sca_kv_shape* shape, int64_t elem_bytes, void* stream) {
    int64_t row_bytes = 0;
    int rc = sca_hip::CheckShape(shape, elem_bytes, "kv_gather", &row_bytes);
    if (rc != 0) return rc;
    if (num_block_ids <= 0) return 0;
    if (layer == nullptr || block_ids == nullptr || out == nullptr) {
        return SetError(SCA_E_SHAPE_MISMATCH, "kv_gather: null pointer");
    }
    if (!sca_hip::Aligned16(layer) || !sca_hip::Aligned16(out)) {
        return SetError(SCA_E_LAYOUT_MISMATCH, "kv_gather: buffers must be 16 B aligned");
    }
    const int64_t block_chunks = row_bytes * shape->block_size / 16;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(sca_hip::kv_gather_kernel,
                       dim3(sca_hip::GridFor(num_block_ids * block_chunks)),
                       dim3(sca_hip::kThreads), 0, s, static_cast<const uint4*>(layer), block_ids,
                       num_block_ids, static_cast<uint4*>(out), block_chunks, shape->num_blocks);
    return sca_hip::CheckLaunch("kv_gather_kernel", s);
}

int sca_hip_i32_scatter(int32_t* dst, int64_t dst_len, const int32_t* pairs, int64_t num_pairs,
                        void* stream) {
    if (num_pairs <= 0) return 0;
    if (dst == nullptr || pairs == nullptr) {
        return SetError(SCA_E_SHAPE_MISMATCH, "i32_scatter: null pointer");
    }
    if ((reinterpret_cast<uintptr_t>(pairs) & 7u) != 0) {
        return SetError(SCA_E_LAYOUT_MISMATCH, "i32_scatter: pairs must be 8 B aligned");
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(sca_hip::i32_scatter_kernel, dim3(sca_hip::GridFor(num_pairs)),
                       dim3(sca_hip::kThreads), 0, s, dst, dst_len,
                       reinterpret_cast<const int2*>(pairs), num_pairs);
    return sca_hip::CheckLaunch("i32_scatter_kernel", s);
}

}  // extern "C"
