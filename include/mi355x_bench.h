/*
 * mi355x_bench.h - C ABI of libmi355x_bench.so, the gfx950 (AMD Instinct
 * MI355X) kernels behind the peak-throughput suite.
 *
 * The reference suite launches Triton kernels through `kernel[grid](...)` and
 * reads compiled-kernel metadata from the returned object. This library
 * replaces that boundary with plain C entry points that take device pointers,
 * sizes and a HIP stream (passed as `void*`, NULL = the default stream).
 * Each declaration names the reference interface it replaces.
 *
 * Conventions:
 *   - return MB_OK (0) on success, a negative MB_ERR_* code on failure, and
 *     never abort, throw or exit; mb_last_error() returns the message of the
 *     calling thread's most recent failure;
 *   - all device memory is allocated and owned by the caller;
 *   - launches are asynchronous on `stream`; nothing here synchronises;
 *   - one launch = one pass of the kernel over the caller's buffers.
 */
#ifndef MI355X_BENCH_H
#define MI355X_BENCH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Version 2: mb_gemm takes MXFP4 scales in K-step blocks [ceil(k/256)][rows][8]
 * (version 1 took them row-major, [rows][k/32]). The two have the same byte
 * count when k is a multiple of 256, so a caller built for version 1 must not
 * load this library: check mb_abi_version() first. */
#define MB_ABI_VERSION 2

#define MB_OK 0
#define MB_ERR_INVALID (-1)     /* bad argument: size, shape, configuration */
#define MB_ERR_UNSUPPORTED (-2) /* valid request this library has no path for */
#define MB_ERR_HIP (-3)         /* the HIP runtime reported an error */
#define MB_ERR_ALIGNMENT (-4)   /* pointer alignment does not fit the kernel */

/* ---- library and device ------------------------------------------------- */

/* ABI version of the loaded library (MB_ABI_VERSION at build time). */
int mb_abi_version(void);

/* Message describing the calling thread's most recent failure ("" if none). */
const char* mb_last_error(void);

typedef struct mb_device_info {
  char name[256];           /* marketing name (hipDeviceProp_t.name) */
  char arch[64];            /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int32_t compute_units;    /* multiProcessorCount */
  int32_t wavefront_size;   /* 64 on CDNA */
  int32_t clock_khz;        /* peak engine clock reported by the runtime */
  int32_t memory_clock_khz; /* memory clock reported by the runtime */
  int32_t memory_bus_bits;  /* memory bus width */
  int32_t reserved0;
  int64_t l2_cache_bytes;   /* L2 size as HIP reports it (one XCD's L2) */
  int64_t lds_bytes_per_cu; /* maxSharedMemoryPerMultiProcessor */
  int64_t total_memory_bytes; /* hipMemGetInfo total */
  int64_t free_memory_bytes;  /* hipMemGetInfo free */
} mb_device_info;

/* Device metadata for the setup block of every result document.
 * Replaces: common.py:214-292 (setup_device) and bench_suite.py:106-114
 * (probe_device), which read torch/Triton device properties and fall back to
 * mem_get_info() for total memory (common.py:254-259). */
int mb_device_query(int device, mb_device_info* out);

typedef struct mb_kernel_attributes {
  int32_t registers_per_thread; /* hipFuncAttributes.numRegs */
  int32_t max_threads_per_block;
  int64_t lds_bytes;            /* static group segment (sharedSizeBytes) */
  int64_t scratch_bytes;        /* private segment per lane (localSizeBytes) */
} mb_kernel_attributes;

/* Number of registered kernels and their stable names. */
int mb_kernel_count(void);
const char* mb_kernel_name(int index);

/* Runtime attributes of a registered kernel. Replaces the Triton
 * CompiledKernel metadata the reference audits: n_regs, n_spills and
 * metadata.shared (bench_tensor.py:1134-1136, bench_vector.py:625-627). */
int mb_kernel_attributes_query(const char* name, mb_kernel_attributes* out);

/* ---- engine clock -------------------------------------------------------- */

/* Rate of the device's constant real-time counter (hipDeviceAttributeWallClockRate) of the current device, in kHz. */
int mb_wall_clock_khz(int* khz);

/* Launches one wave on `stream` that measures the engine clock of its CU over
 * `microseconds` (1..10^7) of real time while other work runs: out[0] =
 * shader clock cycles (s_memtime), out[1] = real-time counter ticks
 * (s_memrealtime) over the same interval, out[2] = polls made, out[3] = the
 * real-time counter at the start. clock in kHz = out[0] / out[1] *
 * mb_wall_clock_khz. `out` holds 4 uint64 in device memory. The wave sleeps
 * between polls; the loop also ends after a bounded number of polls, so
 * out[1] below the requested interval means it ended early.
 * No counterpart in the reference (its rows report no clock); it serves the
 * headline benchmark, which records the clock each row's kernel ran at. */
int mb_clock_witness(uint64_t* out, uint64_t out_bytes, uint32_t microseconds, void* stream);

/* ---- memory: copy and read ---------------------------------------------- */

/* Flags for mb_copy. */
#define MB_COPY_NONTEMPORAL 1u   /* streaming (nt) loads; nt stores unless MB_COPY_WRITE_THROUGH */
#define MB_COPY_WRITE_THROUGH 2u /* device-scope (sc1) stores, written through the XCD's L2 */

/* dst[0:bytes) = src[0:bytes): a coalesced 16-byte-per-lane copy.
 * `block_threads` is a multiple of 64 up to 1024; each workgroup moves
 * `block_threads * vectors_per_thread * 16` bytes per step. `grid_blocks` = 0
 * launches one workgroup per step (the reference's grid = cdiv(N, BLOCK));
 * otherwise that many workgroups stride over the buffer. A tail shorter than
 * 16 bytes, or pointers without 16-byte alignment, take narrower accesses.
 * Replaces: bench_bandwidth.py:36-47 (copy_kernel, launch_copy). */
int mb_copy(const void* src, void* dst, uint64_t bytes, uint32_t block_threads,
            uint32_t vectors_per_thread, uint32_t grid_blocks, uint32_t flags, void* stream);

/* Every 32-bit word of dst[0:bytes) = `pattern` (byte i of a tail shorter
 * than 16 bytes = byte i % 4 of the little-endian pattern): the copy's store
 * stream alone, one 16-byte store per lane, `flags` as for mb_copy (store
 * policy only). dst must be 16-byte aligned. `grid_blocks` = 0 launches one
 * workgroup per `block_threads` vectors; otherwise that many stride over dst.
 * No counterpart in the reference, which measures copy and read only: with
 * mb_read_sum it gives the write-only and read-only HBM rates that bound a
 * copy, which mixes the two. */
int mb_fill(void* dst, uint64_t bytes, uint32_t pattern, uint32_t block_threads, uint32_t grid_blocks,
            uint32_t flags, void* stream);

/* Element types understood by mb_read_sum. */
#define MB_DTYPE_F32 0
#define MB_DTYPE_F16 1
#define MB_DTYPE_BF16 2

/* sink[i] = sum(float(src[i*block_elements : (i+1)*block_elements])), the last
 * segment clipped at `elements`; sink has cdiv(elements, block_elements)
 * float32 entries. `block_elements` is a power of two between 64 and 65536.
 * Replaces: bench_bandwidth.py:50-67 (read_kernel, launch_read). */
int mb_read_sum(int dtype, const void* src, float* sink, uint64_t elements,
                uint32_t block_elements, uint32_t block_threads, void* stream);

/* ---- tensor: resident-operand matrix peak ------------------------------- */

/* Matrix operand formats. */
#define MB_MATRIX_BF16 0
#define MB_MATRIX_F16 1
#define MB_MATRIX_F32 2      /* IEEE fp32 operands, v_mfma_f32_32x32x2_f32 */
#define MB_MATRIX_TF32 3     /* always MB_ERR_UNSUPPORTED: gfx950 has no xf32 MFMA */
#define MB_MATRIX_I8 4       /* int8 operands, int32 accumulate */
#define MB_MATRIX_F64 5      /* fp64 operands and accumulate */
#define MB_MATRIX_FP8_E4M3 6 /* OCP FP8 E4M3 (fn) operands, fp32 accumulate */
#define MB_MATRIX_MXFP4 7    /* OCP MX FP4: E2M1 two per byte + E8M0 scale per 32 K */

typedef struct mb_peak_config {
  uint32_t tile_m;  /* rows of A and C per workgroup */
  uint32_t tile_n;  /* columns of B and C per workgroup */
  uint32_t tile_k;  /* reduction length in elements (E2M1 elements for MXFP4) */
  uint32_t chains;  /* independent accumulators, one B operand each */
  uint32_t b_nk;    /* 0: B tile stored [K][N] (N contiguous); 1: [N][K] */
  uint32_t mfma_m;  /* MFMA output rows (32 or 16) selecting the instruction; 0 = first match */
  uint32_t threads; /* workgroup size (output only) */
} mb_peak_config;

/* Tile configurations compiled for `format`; writes up to `capacity` entries
 * to `out` (which may be NULL) and returns how many exist. */
int mb_tensor_peak_configs(int format, mb_peak_config* out, int capacity);

/* Registered kernel name of a configuration (for the instruction audit), or
 * NULL when no such kernel exists. */
const char* mb_tensor_peak_kernel_name(int format, const mb_peak_config* config);

/* Resident-operand peak: workgroup w computes, for each chain c,
 *   C[c][w] = iterations * (A[w] . B[c][w])
 * in the format's accumulator (fp32; int32 for I8; fp64 for F64), reading its
 * operands from HBM once. Layouts (row-major, all contiguous):
 *   A [blocks][tile_m][tile_k]            (MXFP4: [tile_k/2] bytes, low nibble = even k)
 *   B [chains][blocks][tile_k][tile_n]    (b_nk: [chains][blocks][tile_n][tile_k];
 *                                          MXFP4 [tile_k/2][tile_n] packed along K)
 *   scale_a [blocks][tile_m][tile_k/32], scale_b [blocks][tile_n][tile_k/32] (MXFP4 only)
 *   C [chains][blocks][tile_m][tile_n]
 * Buffer sizes are checked against the configuration before launching.
 * Replaces: bench_tensor.py:406-449 (_tensor_peak_kernel), 452-488
 * (_tensor_peak_scaled_kernel) and 581-600 (_launch_peak). */
int mb_tensor_peak(int format, const mb_peak_config* config, const void* a, uint64_t a_bytes,
                   const void* b, uint64_t b_bytes, const void* scale_a, uint64_t scale_a_bytes,
                   const void* scale_b, uint64_t scale_b_bytes, void* c, uint64_t c_bytes,
                   uint32_t blocks, uint32_t iterations, void* stream);

/* ---- tensor: dense GEMM ---------------------------------------------------- */

typedef struct mb_gemm_config {
  uint32_t tile_m;  /* output rows per workgroup */
  uint32_t tile_n;  /* output columns per workgroup */
  uint32_t tile_k;  /* K elements staged through LDS per step */
  uint32_t threads; /* workgroup size (output only) */
} mb_gemm_config;

/* Tile configurations compiled for `format` (see mb_tensor_peak_configs). */
int mb_gemm_configs(int format, mb_gemm_config* out, int capacity);

/* Registered kernel name of a GEMM configuration, or NULL. */
const char* mb_gemm_kernel_name(int format, const mb_gemm_config* config);

/* C = A . B with A row-major [m][k] and B column-major, i.e. stored [n][k]
 * (both K-contiguous); C row-major [m][n] in the format's accumulator type
 * (fp32; int32 for I8; fp64 for F64). MXFP4: A and B hold two E2M1 codes per
 * byte along K (even k in the low nibble); scale_a and scale_b are E8M0 in
 * K-step blocks, [ceil(k/256)][m][8] and [ceil(k/256)][n][8] bytes, where
 * [b][r][g] scales row r over K elements 256b+32g .. 256b+32g+31 (entries
 * past K are ignored): one 256-element K step of a tile reads one contiguous
 * run of 8 bytes per row. K * element bits must be a multiple of 128 (16-byte
 * rows); other shapes are bounded by a checked kernel variant. group_m = 0
 * selects the variant's default band height (tile rows per band: 8, or the
 * measured best of its fast-path kernel: 4 for BF16 and FP16, 6 for FP8 and 7
 * for INT8 256x256);
 * a band taller than the tile rows acts as the full height. The band height
 * orders the tiles only: every value gives the same C.
 * Replaces: bench_tensor.py:172-209 (_gemm_kernel) and 235-246 (_launch),
 * whose B is row-major [k][n]; the reference has no MXFP4 GEMM (FP4 is refused
 * in its GEMM mode, bench_tensor.py:1404-1407), so the scale layout is this
 * library's. */
int mb_gemm(int format, const mb_gemm_config* config, const void* a, uint64_t a_bytes, const void* b,
            uint64_t b_bytes, const void* scale_a, uint64_t scale_a_bytes, const void* scale_b,
            uint64_t scale_b_bytes, void* c, uint64_t c_bytes, uint32_t m, uint32_t n, uint32_t k,
            uint32_t group_m, void* stream);

/* Registered name of the kernel mb_gemm launches for this call (the tile's
 * fast kernel, or its "_checked" variant for shapes the fast kernel does not
 * take), for the instruction and resource audit of what actually runs; NULL
 * with mb_last_error() set for an invalid call.
 * Replaces: the CompiledKernel the reference's launch returns for its audit
 * (bench_tensor.py:594-600, 988). */
const char* mb_gemm_launched_kernel(int format, const mb_gemm_config* config, uint32_t m, uint32_t n, uint32_t k,
                                    const void* scale_a, const void* scale_b);

/* ---- vector: register-resident arithmetic chains ------------------------ */

/* Vector chain kinds. Storage of input/output/coefficients per kind:
 *   F32 float, F64 double, F16 _Float16, BF16_* bfloat16 bits (uint16),
 *   I8_DOT4 int32 (four packed signed bytes of state; weights packed the same). */
#define MB_VECTOR_F32 0       /* x <- fma(x, a, b_c), v_fma_f32 */
#define MB_VECTOR_F16 1       /* x <- fma(x, a, b_c), v_pk_fma_f16 (two chains per VGPR) */
#define MB_VECTOR_BF16_DOT2 2 /* x <- bf16(a*x + b_c), v_dot2_f32_bf16 + v_cvt_pk_bf16_f32 */
#define MB_VECTOR_F64 3       /* x <- fma(x, a, b_c), v_fma_f64 */
#define MB_VECTOR_I8_DOT4 4   /* x <- dot4(bytes(x), bytes(W)) + b_c, v_dot4_i32_i8 */
#define MB_VECTOR_BF16_FMA 5  /* x <- bf16(fma(f32(x), a, b_c)), v_fma_f32 + v_cvt_pk_bf16_f32 */
#define MB_VECTOR_FP8 6       /* always MB_ERR_UNSUPPORTED: no FP8 vector arithmetic on gfx950 */
#define MB_VECTOR_FP4 7       /* always MB_ERR_UNSUPPORTED: no FP4 vector arithmetic on gfx950 */
/* Widened (converted) FP8/FP4 chains, not native arithmetic: the state stays
 * FP8 E4M3 / FP4 E2M1 (one code per byte in memory, a = Coefficients[0] and
 * b_c = Coefficients[1+c] as codes too) and every update is
 *   x <- narrow(fma(f32(x), f32(a), f32(b_c)))
 * with v_cvt_pk_f32_fp8 / v_cvt_scalef32_pk_f32_fp4 (scale 1) widening a pair
 * of chains, two v_fma_f32, and v_cvt_pk_fp8_f32 / v_cvt_scalef32_pk_fp4_f32
 * rounding the pair back (round to nearest even). They replace the
 * reference's Ascend C converted vector rows (ascendc/src/bench_vector.asc:335-572). */
#define MB_VECTOR_FP8_WIDENED 8
#define MB_VECTOR_FP4_WIDENED 9

/* Registered kernel name of (kind, unroll), or NULL. */
const char* mb_vector_kernel_name(int kind, uint32_t unroll);

/* Eight independent chains per element: for c in 0..7 and every element i,
 *   Output[c][i] = update^iterations(Input[c][i]) with a = Coefficients[0] (for
 *   I8_DOT4 the packed weights W) and b_c = Coefficients[1 + c].
 * One thread per element: `elements` is a positive multiple of
 * `block_threads` (a multiple of 64 up to 1024); the loop body applies
 * `unroll` (1, 4, 8 or 16) updates per trip and `iterations` must be a
 * multiple of it. Buffer sizes are checked before launching.
 * Replaces: bench_vector.py:182-319 (vector_fma_kernel, with _float_update,
 * _widened_fma_update and _dp4a_update) and 1032-1051 (launch_vector). */
int mb_vector_chains(int kind, const void* input, void* output, const void* coefficients,
                     uint64_t elements, uint32_t iterations, uint32_t unroll, uint32_t block_threads,
                     uint64_t input_bytes, uint64_t output_bytes, uint64_t coefficient_bytes,
                     void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MI355X_BENCH_H */
