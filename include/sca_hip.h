/*
 * sca_hip.h - C ABI of the MI355X (gfx950) kernel library `libsca_hip.so`.
 *
 * This is the only header through which host code reaches the GPU. Every HIP runtime call and
 * every kernel launch of the attention stack lives behind these functions; the C++ host layer
 * (sca:: API, dispatcher, KV cache) and any foreign-language binding (ctypes, cgo, JNI) call them
 * with plain pointers, sizes and POD structs. No C++ or framework types cross this boundary.
 *
 * Conventions
 *   - Every function returning `int` returns 0 on success. A positive value below 2000 is a
 *     hipError_t; 2001..2010 are the attention status codes (SCA_E_*); the text of the last
 *     failure on the calling thread is available from sca_hip_last_error_string().
 *   - Pointers named q/k/v/out/lse/partial_* / page_table / seq_lens / slot_mapping /
 *     block_ids are device pointers and are borrowed for the duration of the (asynchronous)
 *     launch. Scratch (split-K partials) is always caller-provided: the library allocates no
 *     device memory on any launch path.
 *   - `stream` is a hipStream_t passed as void*; NULL means the default stream.
 *   - Thread-compatible: concurrent calls on different streams are safe; the library keeps no
 *     mutable device state.
 *
 * Each launch entry point replaces one device-side entry point of the reference
 * (DeRuiChen258/SciCompute-Attention); the replaced declaration is cited above each function.
 */
#ifndef SCA_HIP_H_
#define SCA_HIP_H_

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define SCA_HIP_API __attribute__((visibility("default")))
#else
#define SCA_HIP_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------------------------- */
/* status codes                                                                                 */
/* ------------------------------------------------------------------------------------------- */
enum {
    SCA_OK = 0,
    SCA_E_UNSUPPORTED_HEAD_DIM = 2001,
    SCA_E_UNSUPPORTED_DTYPE = 2002,
    SCA_E_UNSUPPORTED_LAYOUT = 2003,
    SCA_E_LAYOUT_MISMATCH = 2004,
    SCA_E_SHAPE_MISMATCH = 2005,
    SCA_E_SEQ_TOO_LONG = 2006,
    SCA_E_KV_CAPACITY = 2007,
    SCA_E_WORKSPACE = 2008,
    SCA_E_UNSUPPORTED_FEATURE = 2009,
    SCA_E_DEVICE_CAPABILITY = 2010
};

/* Element type of Q/K/V/O (the compute dtype ids of the reference's launchers). */
enum { SCA_DTYPE_F32 = 0, SCA_DTYPE_F16 = 1, SCA_DTYPE_BF16 = 2 };

/* Message of the last failing call on this thread ("" when none). Never NULL. */
SCA_HIP_API const char* sca_hip_last_error_string(void);

/* ------------------------------------------------------------------------------------------- */
/* device probe                                                                                 */
/* replaces: src/runtime/device_probe.h:14-36 (ScaDeviceProbe, sca_probe_device,                */
/*           sca_mem_get_info)                                                                  */
/* ------------------------------------------------------------------------------------------- */
#define SCA_HIP_DEVICE_NAME_MAX 256

typedef struct ScaHipDeviceProbe {
    char name[SCA_HIP_DEVICE_NAME_MAX];
    char arch_name[64];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int major;
    int minor;
    int cu_count;                /* multiProcessorCount (compute units) */
    int wave_size;               /* 64 on CDNA */
    int clock_khz;               /* peak shader clock */
    int memory_clock_khz;
    int memory_bus_width_bits;
    unsigned long long lds_per_cu;             /* maxSharedMemoryPerMultiProcessor */
    unsigned long long lds_per_block;          /* sharedMemPerBlock */
    unsigned long long regs_per_cu;
    unsigned long long max_threads_per_cu;
    unsigned long long l2_bytes;
    unsigned long long total_mem_bytes;
    unsigned long long free_mem_bytes;
    int gpu_available;           /* 1 when a HIP device was found */
    int binary_has_gfx950;       /* this library carries gfx950 code objects (MFMA f16/bf16 K=16) */
} ScaHipDeviceProbe;

SCA_HIP_API int sca_hip_probe_device(int device_id, ScaHipDeviceProbe* out);
SCA_HIP_API int sca_hip_mem_get_info(unsigned long long* free_bytes,
                                     unsigned long long* total_bytes);
SCA_HIP_API int sca_hip_get_device_count(int* count);

/* ------------------------------------------------------------------------------------------- */
/* memory, streams, events (the plumbing the host layer's sci::Device/Stream use)               */
/* ------------------------------------------------------------------------------------------- */
enum { SCA_COPY_H2D = 1, SCA_COPY_D2H = 2, SCA_COPY_D2D = 3, SCA_COPY_H2H = 4 };

SCA_HIP_API int sca_hip_malloc(void** ptr, size_t bytes);
SCA_HIP_API int sca_hip_free(void* ptr);
SCA_HIP_API int sca_hip_host_malloc(void** ptr, size_t bytes); /* pinned host memory */
SCA_HIP_API int sca_hip_host_free(void* ptr);
SCA_HIP_API int sca_hip_memcpy(void* dst, const void* src, size_t bytes, int kind);
SCA_HIP_API int sca_hip_memcpy_async(void* dst, const void* src, size_t bytes, int kind,
                                     void* stream);
/* Zero-fill with a kernel (graph-capture safe, unlike a memset node). */
SCA_HIP_API int sca_hip_zero_async(void* ptr, size_t bytes, void* stream);
SCA_HIP_API int sca_hip_device_synchronize(void);
SCA_HIP_API int sca_hip_stream_create(void** stream);
SCA_HIP_API int sca_hip_stream_destroy(void* stream);
SCA_HIP_API int sca_hip_stream_synchronize(void* stream);
SCA_HIP_API int sca_hip_event_create(void** event);
SCA_HIP_API int sca_hip_event_destroy(void* event);
SCA_HIP_API int sca_hip_event_record(void* event, void* stream);
SCA_HIP_API int sca_hip_event_synchronize(void* event);
SCA_HIP_API int sca_hip_event_elapsed_ms(float* ms, void* start, void* stop);

/* ------------------------------------------------------------------------------------------- */
/* flash prefill                                                                                */
/* replaces: src/backends/flash/flash_fwd_kernel.cuh:32-60 (FlashFwdParams, FlashSmemBytesFor,  */
/*           LaunchFlashFwd)                                                                    */
/* ------------------------------------------------------------------------------------------- */
typedef struct sca_flash_params {
    const void* q;       /* element (b,h,s,d) at b*q_sb + h*q_sh + s*q_ss + d */
    const void* k;
    const void* v;
    void* out;
    float* lse;          /* optional FP32 [b,h,s] at (b*num_heads + h)*seq_q + s; NULL = none */
    int64_t batch;
    int64_t num_heads;   /* H_q */
    int64_t num_kv_heads;/* H_kv; H_q % H_kv == 0, kv head = h / (H_q/H_kv) */
    int64_t seq_q;
    int64_t seq_kv;
    int64_t head_dim;    /* 32, 64, 96, 128, 160, 192 or 256 */
    int64_t q_sb, q_sh, q_ss;
    int64_t k_sb, k_sh, k_ss;
    int64_t v_sb, v_sh, v_ss;
    int64_t o_sb, o_sh, o_ss;
    float scale;         /* softmax scale (already resolved, > 0) */
    int32_t causal;      /* bottom-right aligned: key j visible from row i iff j <= i + diagonal */
    int32_t dtype;       /* SCA_DTYPE_F16 or SCA_DTYPE_BF16 */
    int64_t diagonal;    /* seq_kv - seq_q when causal */
} sca_flash_params;

/* LDS bytes one workgroup of the flash kernel uses for this head_dim (-1 if not built). */
SCA_HIP_API int64_t sca_hip_flash_lds_bytes(int32_t head_dim, int64_t elem_bytes);
/* Tile geometry of the flash kernel for head_dim: rows per workgroup, keys per tile, waves. */
SCA_HIP_API int sca_hip_flash_tile(int32_t head_dim, int32_t* block_m, int32_t* block_n,
                                   int32_t* waves, int32_t* stages);
SCA_HIP_API int sca_hip_flash_fwd(const sca_flash_params* params, void* stream);

/* Packed variable-length prefill in one launch (no reference counterpart: the reference's
 * FlashBackend::ForwardVarlen, flash_backend.cpp:226-376, launches once per sequence).
 * q/out are packed [T_q, H_q, D] and k/v [T_kv, H_kv, D] (token stride *_ss, head stride *_sh);
 * sequence s spans tokens [cu_seqlens_q[s], cu_seqlens_q[s+1]) and likewise for k/v. `tiles` is
 * the device copy of the work list sca_hip_flash_varlen_tiles writes (2 int32 per 128-row tile:
 * sequence, row tile; longest first). head_dim 64 or 128 (other head dims: launch per sequence).
 * Causal masking is bottom-right per sequence (key j visible from row i iff j <= i + S_kv - S_q). */
typedef struct sca_flash_varlen_params {
    const void* q;
    const void* k;
    const void* v;
    void* out;
    const int32_t* cu_seqlens_q;  /* device, num_seqs + 1 */
    const int32_t* cu_seqlens_kv; /* device, num_seqs + 1 */
    const int32_t* tiles;         /* device, 2 * num_tiles */
    int64_t num_seqs;
    int64_t num_tiles;
    int64_t max_seq_kv;
    int64_t num_heads;
    int64_t num_kv_heads;
    int64_t head_dim;
    int64_t q_sh, q_ss;
    int64_t k_sh, k_ss;
    int64_t v_sh, v_ss;
    int64_t o_sh, o_ss;
    float scale;
    int32_t causal;
    int32_t dtype;                /* SCA_DTYPE_F16 or SCA_DTYPE_BF16 */
} sca_flash_varlen_params;

/* Work list of a packed launch from host cu_seqlens: writes 2 int32 per row tile (sequence, tile)
 * into tiles_out (may be NULL to count only), ordered by decreasing key count; returns the tile
 * count, or a negative status when the lengths are invalid. */
SCA_HIP_API int64_t sca_hip_flash_varlen_tiles(const int32_t* cu_seqlens_q,
                                               const int32_t* cu_seqlens_kv, int64_t num_seqs,
                                               int32_t causal, int32_t* tiles_out);
/* 1 when head_dim has the one-launch varlen kernel. */
SCA_HIP_API int sca_hip_flash_varlen_supported(int32_t head_dim);
SCA_HIP_API int sca_hip_flash_fwd_varlen(const sca_flash_varlen_params* params, void* stream);

/* ------------------------------------------------------------------------------------------- */
/* split-K decode (contiguous and paged)                                                        */
/* replaces: src/backends/decode/decode_splitk.cuh:15-57 (DecodeFwdParams, LaunchDecodeSplitK,  */
/*           LaunchDecodeSplitKPaged) and src/backends/paged/paged_attention.cuh:21-32          */
/*           (LaunchPagedAttention)                                                             */
/* ------------------------------------------------------------------------------------------- */
typedef struct sca_decode_params {
    const void* q;        /* one query token per (b, h): element at b*q_sb + h*q_sh + d */
    const void* k;        /* contiguous: b*k_sb + h_kv*k_sh + j*k_ss + d;                  */
    const void* v;        /* paged: layer base, row r at r*k_ss + h_kv*k_sh + d            */
    void* out;            /* element at b*o_sb + h*o_sh + d */
    float* partial_m;     /* [batch*num_heads*num_splits], flat ((b*H_q)+h)*splits + s */
    float* partial_l;     /* same indexing */
    float* partial_o;     /* [batch*num_heads*num_splits, head_dim] */
    int64_t batch;
    int64_t num_heads;
    int64_t num_kv_heads;
    int64_t seq_kv;       /* contiguous length, or the upper bound when seq_lens is NULL */
    int64_t head_dim;     /* multiple of 32, <= 256 */
    int64_t num_splits;   /* >= 1 */
    int64_t q_sb, q_sh;
    int64_t k_sb, k_sh, k_ss;
    int64_t v_sb, v_sh, v_ss;
    int64_t o_sb, o_sh;
    float scale;
    int32_t dtype;        /* SCA_DTYPE_F32, F16 or BF16 */
    /* paged addressing (page_table != NULL): row = page_table[b*max_blocks_per_seq + j/bs]*bs
     * + j%bs; entries < 0 or >= num_kv_blocks contribute nothing */
    const int32_t* page_table;
    int64_t block_size;
    int64_t max_blocks_per_seq;
    int64_t num_kv_blocks;
    const int32_t* seq_lens; /* optional per-sequence lengths (device), else seq_kv for all */
    /* optional device scratch of 2*batch int32 (8-byte aligned). With seq_lens set, sequences
     * are scheduled longest first; batches of up to 256 sequences are ranked inside the kernel,
     * larger ones (up to 8192) through this scratch (no reference counterpart: the reference
     * launches sequences in batch order). NULL = batch order above 256 sequences. */
    int32_t* batch_order;
    /* MFMA kernel work split for fp16/bf16 with head_dim 64 or 128 (no reference counterpart):
     * 0 = library default (one wave per KV-head slot for paged KV, four for contiguous),
     * 1 = one wave per slot (a workgroup serves four slots), 4 = four waves per slot (a
     * workgroup serves one slot and its waves share the key tiles). Other values are rejected.
     * Results agree either way to FP32 rounding of the merge; a planner picks the faster one
     * per batch (sca_paged_decode_plan). */
    int32_t slot_waves;
} sca_decode_params;

/* FP32 scratch elements the partials need: batch*num_heads*num_splits*(2 + head_dim). */
SCA_HIP_API int64_t sca_hip_decode_partial_elements(int64_t batch, int64_t num_heads,
                                                    int64_t num_splits, int64_t head_dim);
SCA_HIP_API int sca_hip_decode_splitk(const sca_decode_params* params, void* stream);
SCA_HIP_API int sca_hip_decode_splitk_paged(const sca_decode_params* params, void* stream);
/* Allocation-free variant of sca_hip_decode_splitk (contiguous or paged, as page_table says).
 * No counterpart in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). partial_m/l/o
 * and batch_order must be NULL: the split partials (at most 16 MiB:
 * 4*sca_hip_decode_partial_elements(...) bytes) and the ranking scratch live in a static device
 * array, one per GPU the library is loaded on (reserved for every process that loads it, used
 * or not), held until the process ends. Larger split counts fail with
 * SCA_E_WORKSPACE. Every call on one GPU shares that array: calls that overlap on one GPU (on
 * different streams) race; calls ordered on one stream are safe. */
SCA_HIP_API int sca_hip_decode_splitk_noalloc(const sca_decode_params* params, void* stream);

/* ------------------------------------------------------------------------------------------- */
/* KV cache data movement over the block-major layout [num_blocks][block_size][H_kv][D]         */
/* replaces: src/kv_cache/kv_cache_kernels.cuh:20-33 (LaunchKvAppend, LaunchKvResetBlock,       */
/*           LaunchKvGather)                                                                    */
/* ------------------------------------------------------------------------------------------- */
typedef struct sca_kv_shape {
    int64_t num_blocks;
    int64_t block_size;
    int64_t num_kv_heads;
    int64_t head_dim;
} sca_kv_shape;

/* dst row `slot` of K and V <- row t of k_new/v_new ([num_tokens, H_kv, D]); slot < 0 or a block
 * beyond num_blocks skips the token. */
SCA_HIP_API int sca_hip_kv_append(void* layer_k, void* layer_v, const void* k_new,
                                  const void* v_new, const int32_t* slot_mapping,
                                  int64_t num_tokens, const sca_kv_shape* shape,
                                  int64_t elem_bytes, void* stream);
/* Zeroes K and V of the listed blocks (ids outside [0, num_blocks) are skipped). */
SCA_HIP_API int sca_hip_kv_reset_blocks(void* layer_k, void* layer_v, const int32_t* block_ids,
                                        int64_t num_block_ids, const sca_kv_shape* shape,
                                        int64_t elem_bytes, void* stream);
/* out[i] <- block block_ids[i] of `layer` (out is [n, block_size, H_kv, D]); invalid ids give
 * zero rows. */
SCA_HIP_API int sca_hip_kv_gather(const void* layer, const int32_t* block_ids,
                                  int64_t num_block_ids, void* out, const sca_kv_shape* shape,
                                  int64_t elem_bytes, void* stream);

/* Sparse int32 update: dst[pairs[2i]] = pairs[2i+1] for i < num_pairs (indices outside
 * [0, dst_len) are skipped; pairs 8 B aligned, device). Used to refresh only the changed entries
 * of a device page table.
 * replaces: the whole-table re-upload of src/kv_cache/paged_kv_cache.cpp:182-201 (no kernel
 *           counterpart in the reference) */
SCA_HIP_API int sca_hip_i32_scatter(int32_t* dst, int64_t dst_len, const int32_t* pairs,
                                    int64_t num_pairs, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SCA_HIP_H_ */
