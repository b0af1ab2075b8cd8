// Device-side helpers shared by the gfx950 kernels: vector types for the MFMA operands, dtype
// conversion, cross-lane helpers and the thread-local error text of the C ABI.
//
// Written for CDNA4 (wave64, MFMA f32_32x32x16_{f16,bf16}); there is no other target.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <mutex>
#include <string>

#include "sca_hip.h"

namespace sca_hip {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Storage types. Element bits are moved as uint16_t and reinterpreted at the MFMA boundary so
// that the load/store code is shared by fp16 and bf16.
struct F16 {
    using vec8 = half8;
    static __device__ __forceinline__ float to_float(uint16_t bits) {
        return static_cast<float>(__builtin_bit_cast(_Float16, bits));
    }
    // IEEE round-to-nearest-even (v_cvt_f16_f32).
    static __device__ __forceinline__ uint16_t from_float(float x) {
        return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
    }
};

struct BF16 {
    using vec8 = bf16x8;
    static __device__ __forceinline__ float to_float(uint16_t bits) {
        return __builtin_bit_cast(float, static_cast<uint32_t>(bits) << 16);
    }
    // Round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950).
    static __device__ __forceinline__ uint16_t from_float(float x) {
        return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
    }
};

struct F32 {
    static __device__ __forceinline__ float to_float(float x) { return x; }
    static __device__ __forceinline__ float from_float(float x) { return x; }
};

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }

// v_exp_f32: 2^x. exp2(-inf) = 0, which keeps masked logits exactly out of every sum.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Swap halves of the wave: lane l receives the value of lane l ^ 32.
__device__ __forceinline__ float xor32(float x) { return __shfl_xor(x, 32); }

// 16-lane butterfly sums (DPP-friendly offsets 8,4,2,1 stay inside one 16-lane row).
__device__ __forceinline__ float row16_sum(float x) {
    x += __shfl_xor(x, 8);
    x += __shfl_xor(x, 4);
    x += __shfl_xor(x, 2);
    x += __shfl_xor(x, 1);
    return x;
}

// Transposed LDS read (ds_read_b64_tr_b16): within each 16-lane group, lane j receives element
// j % 4 of the 8 bytes addressed by lane 4*i + j/4, i = 0..3 (one column over four rows).
template <typename E>
struct TrRead;

template <>
struct TrRead<F16> {
    typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 v4;
    static __device__ __forceinline__ uint2 read(const uint8_t* lds_byte_ptr) {
        const v4 r = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
            (__attribute__((address_space(3))) v4*)(lds_byte_ptr));
        return __builtin_bit_cast(uint2, r);
    }
};

template <>
struct TrRead<BF16> {
    typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 v4;
    static __device__ __forceinline__ uint2 read(const uint8_t* lds_byte_ptr) {
        const v4 r = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (__attribute__((address_space(3))) v4*)(lds_byte_ptr));
        return __builtin_bit_cast(uint2, r);
    }
};

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt bits [3:0] and [15:14]).
template <int N>
__device__ __forceinline__ void WaitVm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

}  // namespace sca_hip

// Error reporting of the C ABI (defined in runtime.hip).
namespace sca_hip {
int SetError(int code, const std::string& message);
int CheckLaunch(const char* what, hipStream_t stream);
int FromHip(hipError_t err, const char* what);

// Raises the dynamic LDS limit of kernel `Kernel` to `bytes` the first time it is launched in
// the process. Safe to call from several threads; a failed attribute call is reported as an
// error and retried on the next launch.
template <auto Kernel>
int EnsureLdsLimit(int bytes, const char* what) {
    static std::atomic<bool> done{false};
    static std::mutex mu;
    if (done.load(std::memory_order_acquire)) return 0;
    std::lock_guard<std::mutex> lock(mu);
    if (done.load(std::memory_order_relaxed)) return 0;
    const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(Kernel),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (err != hipSuccess) {
        (void)hipGetLastError();
        return FromHip(err, what);
    }
    done.store(true, std::memory_order_release);
    return 0;
}
}  // namespace sca_hip
