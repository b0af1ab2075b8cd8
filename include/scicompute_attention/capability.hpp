#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

#include "core/status.hpp"
#include "scicompute_attention/export.hpp"

namespace sca {

// What the GPU offers, probed once per device through the kernel library's C ABI and cached
// (Refresh() re-probes). Field names follow the reference's struct so that caller code compiles
// unchanged; on CDNA "sm" means compute unit and "smem" means LDS.
struct SCI_ATTENTION_API DeviceCapability {
    std::string device_name;
    std::string arch_name;               // e.g. "gfx950:sramecc+:xnack-"
    int major{0};
    int minor{0};
    int sm_count{0};                     // compute units
    int wave_size{0};                    // 64 on CDNA
    int clock_khz{0};
    size_t smem_per_sm{0};               // LDS per CU
    size_t smem_per_block_default{0};    // LDS per workgroup
    size_t smem_per_block_optin{0};      // same as default on CDNA (no opt-in carve-out)
    size_t regs_per_sm{0};
    size_t max_threads_per_sm{0};
    size_t l2_bytes{0};
    size_t total_mem_bytes{0};
    size_t free_mem_bytes{0};
    bool has_mfma_f16_k16{false};        // gfx950 v_mfma_f32_32x32x16_{f16,bf16} in this binary
    // NVIDIA-only features of the reference's struct; always false on this hardware.
    bool has_mma_m16n8k16{false};
    bool has_cp_async{false};
    bool has_tma_bulk{false};
    bool has_wgmma{false};
    bool has_fp8_mma{false};

    static const DeviceCapability& ForDevice(int device_id = 0);
    static sci::Status Refresh(int device_id = 0);

    // LDS ceiling per workgroup, lowered by SCI_ATTENTION_MAX_LDS_BYTES (or the reference's
    // SCI_ATTENTION_MAX_SMEM_BYTES) when set.
    static size_t SmemLimitPerBlock(const DeviceCapability& cap) noexcept;

    // True when a HIP GPU is visible. CudaAvailable() is the reference's spelling.
    static bool GpuAvailable() noexcept;
    static bool CudaAvailable() noexcept { return GpuAvailable(); }
};

}  // namespace sca
