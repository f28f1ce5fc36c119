/*
 * fe2o3_mi355x.h -- C-ABI of libfe2o3_mi355x.so, the MI355X (gfx950)
 * implementation of fe2o3's dense-compute example path.
 *
 * Two groups of entry points:
 *
 *  1. The runtime seam.  fe2o3's Rust host reaches HIP through the raw
 *     `extern "C"` block of crates/fe2o3-hip-sys/src/lib.rs:92-165 plus the
 *     C shim fe2o3HipGetDeviceProperties
 *     (crates/fe2o3-hip-sys/native/device_properties.h:14-26).  This library
 *     exports the same capability set (device, stream, event, memory) as
 *     fe2o3_rt_* functions, and the property shim under its reference name
 *     with the same 312-byte record.
 *
 *  2. One function per typed kernel.  The reference's physical kernel ABI is
 *     one (pointer, length) pair per slice argument, in declaration order,
 *     followed by the scalar arguments
 *     (examples/tiled_gemm_general_v1/hardware-harness/src/lib.rs:578-597).
 *     Each entry point below keeps exactly that order and appends the HIP
 *     stream.  Lengths are element counts, as in the Rust slices.
 *
 * Conventions
 *  - Status: 0 = success; a positive value is the hipError_t HIP returned; a
 *    negative value is a fail-closed validation error (FE2O3_ERR_*).  All
 *    validation happens on the host before any launch, so on a negative
 *    status no output byte has been written (the reference's oracles and
 *    typed launchers fail closed the same way,
 *    crates/fe2o3-host/src/loaded_kernel.rs:563-566).
 *  - Kernel entry points are asynchronous: they enqueue on `stream` (NULL =
 *    the null stream) and return.  The reference's typed launch is
 *    synchronous by design (crates/fe2o3-host/src/loaded_kernel.rs:420-432);
 *    its synchronous behaviour is kept by the host mirror
 *    (fe2o3_amd/kernels.py), which synchronizes the stream after each launch.
 *  - Pointers are device pointers unless stated.  Caller owns all memory; the
 *    library never frees caller memory.  Inputs are never written.
 *  - bf16 values are passed as uint16_t bit patterns (the reference's &[u16]).
 */
#ifndef FE2O3_MI355X_H
#define FE2O3_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------------
 * Negative codes share their values with the CPU oracle's (oracle/
 * fe2o3_oracle.h) wherever the meaning is the same. */
#define FE2O3_OK 0
#define FE2O3_ERR_LENGTH (-2)        /* slice length does not match the shape  */
#define FE2O3_ERR_SHAPE (-3)         /* unsupported shape / profile            */
#define FE2O3_ERR_STRIDE (-4)        /* stride smaller than the row extent     */
#define FE2O3_ERR_NONFINITE (-5)     /* NaN input where the contract rejects it */
#define FE2O3_ERR_WEIGHTS (-14)      /* MoE route-weight pair policy           */
#define FE2O3_ERR_OVERFLOW (-16)     /* extent arithmetic overflows            */
#define FE2O3_ERR_NULL (-19)         /* required pointer is NULL               */
#define FE2O3_ERR_DEVICE (-20)       /* current device is not gfx950           */
#define FE2O3_ERR_ALIGNMENT (-21)    /* pointer misaligned for the fast path   */
#define FE2O3_ERR_WORKSPACE (-22)    /* workspace too small                    */
#define FE2O3_ERR_INJECTED (-23)     /* FE2O3_FAULT_POINT forced a failure     */
#define FE2O3_ERR_M_TAIL (-24)       /* M not a multiple of the 16-row tile    */
#define FE2O3_ERR_N_TAIL (-25)       /* N not a multiple of the 16-column tile */
#define FE2O3_ERR_K_TAIL (-26)       /* K not a multiple of the 16-deep tile   */

/* Human-readable text for any status (HIP codes included).  Never NULL. */
const char *fe2o3_status_string(int32_t status);

/* ---- runtime seam (crates/fe2o3-hip-sys/src/lib.rs:92-165) ---------------- */

/* crates/fe2o3-hip-sys/src/lib.rs:49-60 and native/device_properties.h:14-26:
 * fixed-width, 312-byte, 8-aligned record. */
typedef struct Fe2o3HipDeviceProperties {
  char gcn_arch_name[256];
  int32_t warp_size;
  int32_t max_threads_per_block;
  int32_t max_block_dim[3];
  int32_t max_grid_dim[3];
  uint64_t shared_mem_per_block;
  uint64_t shared_mem_per_block_optin;
  uint64_t architecture_features;
} Fe2o3HipDeviceProperties;

#define FE2O3_HIP_DEVICE_ARCH_HAS_GLOBAL_INT32_ATOMICS (UINT64_C(1) << 0)
#define FE2O3_HIP_DEVICE_ARCH_HAS_SHARED_INT32_ATOMICS (UINT64_C(1) << 1)
#define FE2O3_HIP_DEVICE_ARCH_HAS_GLOBAL_INT64_ATOMICS (UINT64_C(1) << 2)
#define FE2O3_HIP_DEVICE_ARCH_HAS_SHARED_INT64_ATOMICS (UINT64_C(1) << 3)
#define FE2O3_HIP_DEVICE_ARCH_HAS_WARP_VOTE (UINT64_C(1) << 4)
#define FE2O3_HIP_DEVICE_ARCH_HAS_WARP_BALLOT (UINT64_C(1) << 5)
#define FE2O3_HIP_DEVICE_ARCH_HAS_WARP_SHUFFLE (UINT64_C(1) << 6)

/* native/device_properties.c:63-101 (same name and record as the reference). */
int32_t fe2o3HipGetDeviceProperties(int32_t device_id,
                                    Fe2o3HipDeviceProperties *properties);

/* lib.rs:93-96: hipInit / hipGetDeviceCount / hipSetDevice. */
int32_t fe2o3_rt_init(uint32_t flags);
int32_t fe2o3_rt_get_device_count(int32_t *count);
int32_t fe2o3_rt_set_device(int32_t device_id);
int32_t fe2o3_rt_get_device(int32_t *device_id);
/* Figures the measurement harness divides by: compute units, peak shader
 * clock (kHz) and memory clock (kHz) / bus width (bits) of the device. */
int32_t fe2o3_rt_device_rates(int32_t device_id, int32_t *compute_units,
                              int32_t *clock_khz, int32_t *memory_clock_khz,
                              int32_t *memory_bus_bits);
/* Fails with FE2O3_ERR_DEVICE unless the device's arch name starts "gfx950". */
int32_t fe2o3_rt_require_gfx950(int32_t device_id);
/* Non-finite inputs.  The reference's kernels that admit only finite inputs
 * trap, and the fault surfaces when the host synchronizes
 * (examples/moe_top2_v1/src/kernel.rs:126-128,
 * examples/flash_attention_v1/src/kernel.rs:143-146; the row-softmax
 * contract rejects them, examples/row_softmax_v1/src/numerical_contract.rs:149).
 * Here such a kernel (fe2o3_row_softmax_v1, fe2o3_row_softmax,
 * fe2o3_flash_attention_causal_f32_b1_h1_n8_d16_v1, both top-2 routers)
 * writes the sentinel outputs its declaration states, adds 1 to the device's
 * non-finite counter and exits normally; the next successful
 * fe2o3_rt_device_synchronize or fe2o3_rt_stream_synchronize on that device
 * that reads a count it has not reported yet returns FE2O3_ERR_NONFINITE.
 * Nothing ever clears the counter, so a rejection that lands while a
 * synchronize reads it is reported by the next one.  The counter is per
 * device, like the reference's context-wide fault: a synchronize reports what
 * any kernel that finished before it on the device found, whichever stream
 * launched it, once.  Event synchronization does not read it. */
int32_t fe2o3_rt_device_synchronize(void);

/* lib.rs:109-111: hipStreamCreate / Destroy / Synchronize. */
int32_t fe2o3_rt_stream_create(void **stream);
int32_t fe2o3_rt_stream_destroy(void *stream);
int32_t fe2o3_rt_stream_synchronize(void *stream);

/* lib.rs:113-123: hipEvent*. */
int32_t fe2o3_rt_event_create(void **event, uint32_t flags);
int32_t fe2o3_rt_event_destroy(void *event);
int32_t fe2o3_rt_event_record(void *event, void *stream);
int32_t fe2o3_rt_event_synchronize(void *event);
int32_t fe2o3_rt_event_query(void *event);
int32_t fe2o3_rt_event_elapsed_ms(float *milliseconds, void *start, void *stop);

/* lib.rs:125-142: hipMalloc / hipFree / hipHostMalloc / hipHostFree /
 * hipMemcpyAsync / hipMemsetAsync.  kind: 0 H2H, 1 H2D, 2 D2H, 3 D2D,
 * 4 default (lib.rs:84-88). */
int32_t fe2o3_rt_malloc(void **ptr, size_t bytes);
int32_t fe2o3_rt_free(void *ptr);
int32_t fe2o3_rt_host_malloc(void **ptr, size_t bytes);
int32_t fe2o3_rt_host_free(void *ptr);
int32_t fe2o3_rt_memcpy_async(void *dst, const void *src, size_t bytes,
                              uint32_t kind, void *stream);
int32_t fe2o3_rt_memcpy(void *dst, const void *src, size_t bytes, uint32_t kind);
int32_t fe2o3_rt_memset_async(void *dst, int32_t value, size_t bytes, void *stream);

/* lib.rs:144-165: hipModuleLoad / hipModuleLoadData / hipModuleUnload /
 * hipModuleGetFunction / hipModuleLaunchKernel, for callers that load code
 * objects of their own.  Modules and functions are HIP handles passed as
 * opaque pointers; kernel_params is HIP's array of pointers to each
 * argument (or NULL with `extra`).  A NULL out-pointer, name, image or
 * handle returns FE2O3_ERR_NULL without calling HIP; otherwise the HIP
 * status is returned, and *module / *function are NULL on failure. */
int32_t fe2o3_rt_module_load(void **module, const char *file_name);
int32_t fe2o3_rt_module_load_data(void **module, const void *image);
int32_t fe2o3_rt_module_unload(void *module);
int32_t fe2o3_rt_module_get_function(void **function, void *module,
                                     const char *kernel_name);
int32_t fe2o3_rt_module_launch_kernel(void *function, uint32_t grid_dim_x,
                                      uint32_t grid_dim_y, uint32_t grid_dim_z,
                                      uint32_t block_dim_x, uint32_t block_dim_y,
                                      uint32_t block_dim_z, uint32_t shared_mem_bytes,
                                      void *stream, void **kernel_params, void **extra);

/* ---- deterministic synthetic inputs --------------------------------------------
 * Counter-based fills that reproduce, bit for bit, the CPU generators of the
 * test oracle (hash = SplitMix64 finaliser of seed ^ domain ^ index *
 * 0xd6e8feb86659fd93; normal = centred Irwin-Hall sum of twelve 16-bit
 * uniforms * 2^-16; uniform = 24-bit on [-1, 1)).  `scale` is applied with
 * one f32 multiply, then bf16 outputs are RNE-narrowed.  Used by the bench
 * to build inputs in HBM without host traffic. */
int32_t fe2o3_fill_normal_bf16(uint16_t *out, uint64_t n, uint64_t seed,
                               uint64_t domain, float scale, uint64_t first_index,
                               void *stream);
int32_t fe2o3_fill_normal_f32(float *out, uint64_t n, uint64_t seed,
                              uint64_t domain, float scale, uint64_t first_index,
                              void *stream);
int32_t fe2o3_fill_uniform_f32(float *out, uint64_t n, uint64_t seed,
                               uint64_t domain, uint64_t first_index, void *stream);

/* ---- GEMM ---------------------------------------------------------------------- */

/* examples/tiled_gemm_v1/src/kernel.rs:63-67 tiled_gemm_lds_slice1(a: &[u16],
 * b: &[u16], c: DisjointSlice<f32, Blocked<Index1D,16,4>>): the fixed
 * 16x16x16 bf16 tile, A row-major [16,16], B row-major [16(K),16(N)],
 * C row-major f32 [16,16].  Lengths must all be 256. */
int32_t fe2o3_tiled_gemm_lds_slice1_v1(const uint16_t *a, uint64_t a_len,
                                       const uint16_t *b, uint64_t b_len,
                                       float *c, uint64_t c_len, void *stream);

/* The multi-tile LDS GEMM of examples/tiled_gemm_v1 under its checked plan
 * (ShapeV1::checked and plan_v1, examples/tiled_gemm_v1/src/contract.rs:
 * 145-179, 387-427): C[m,n] f32 = A[m,k] bf16 (row-major) * B[k,n] bf16
 * (row-major), fp32 accumulation, one wave64 per 16x16 output tile.  The
 * plan's outcomes, in its order:
 *   m == 0 or n == 0  -> NoDispatchEmptyOutput: FE2O3_OK, nothing launched;
 *                        the three lengths must be 0 (no operand buffers);
 *   byte extents of A, B, C overflowing u64 -> FE2O3_ERR_OVERFLOW;
 *   lengths other than m*k, k*n, m*n -> FE2O3_ERR_LENGTH;
 *   m % 16 -> FE2O3_ERR_M_TAIL; n % 16 -> FE2O3_ERR_N_TAIL;
 *   k == 0 -> HostFillPositiveZero: C is filled with +0 (by a kernel);
 *   k % 16 -> FE2O3_ERR_K_TAIL; 64 * n/16 above u32 -> FE2O3_ERR_OVERFLOW;
 *   otherwise Dispatch.
 * On every error nothing is launched and C is untouched. */
int32_t fe2o3_tiled_gemm_v1(const uint16_t *a, uint64_t a_len,
                            const uint16_t *b, uint64_t b_len, float *c,
                            uint64_t c_len, uint32_t m, uint32_t n, uint32_t k,
                            void *stream);

/* examples/tiled_gemm_general_v1/src/kernel.rs:67-79 tiled_gemm_general_v1:
 * c[r*ldc+j] = alpha * sum_d A[r*lda+d]*B[d*ldb+j] + beta * c[r*ldc+j] for
 * r<m, j<n; nothing else of c is touched.  Slices must cover the accessed
 * extent ((rows-1)*stride + cols); stride must be >= cols for a non-empty
 * operand (kernel.rs:80-89, which traps where this returns an error). */
int32_t fe2o3_tiled_gemm_general_v1(const uint16_t *a, uint64_t a_len,
                                    const uint16_t *b, uint64_t b_len,
                                    float *c, uint64_t c_len, uint32_t m,
                                    uint32_t n, uint32_t k, uint32_t lda,
                                    uint32_t ldb, uint32_t ldc, float alpha,
                                    float beta, void *stream);

/* The same kernel contract and arguments under the reference's second
 * schedule, VectorizedAOnlyBf16GlobalTransferV1
 * (crates/dialect-schedule/src/general_gemm.rs:13-38; the hardware harness
 * runs both schedules on the same seven profiles,
 * examples/tiled_gemm_general_v1/hardware-harness/src/lib.rs:135-253): A is
 * staged with one 8-byte load per full, in-range, 8-byte-aligned group of 4
 * elements and masked scalar loads elsewhere; B stays scalar.  Results are
 * bit-identical to fe2o3_tiled_gemm_general_v1. */
int32_t fe2o3_tiled_gemm_general_vector_a_v1(const uint16_t *a, uint64_t a_len,
                                             const uint16_t *b, uint64_t b_len,
                                             float *c, uint64_t c_len, uint32_t m,
                                             uint32_t n, uint32_t k, uint32_t lda,
                                             uint32_t ldb, uint32_t ldc, float alpha,
                                             float beta, void *stream);

/* examples/scalar_gemm_v1/src/kernel.rs:8 scalar_gemm_v1(a: &[f32], b: &[f32],
 * c: DisjointSlice<f32>, m, n, k): row-major f32 C[m,n] = A[m,k] * B[k,n]
 * with the reference's per-output sequential, unfused recurrence
 * (acc = +0; for t in 0..k: acc = acc + a*b, each op separately rounded), so
 * results are bit-identical to the scalar oracle.  Lengths: a >= m*k,
 * b >= k*n, c >= m*n (kernel.rs:8-28 bounds each access by the extents). */
int32_t fe2o3_scalar_gemm_v1(const float *a, uint64_t a_len, const float *b,
                             uint64_t b_len, float *c, uint64_t c_len,
                             uint32_t m, uint32_t n, uint32_t k, void *stream);

/* Scaled-up bf16 GEMM of the BASELINE configuration, generalising
 * tiled_gemm_general_v1 to the MI355X shape: C[m,n] (bf16, row-major) =
 * A[m,k] (bf16, row-major) * B^T where B is stored column-major, i.e. as
 * [n,k] with k contiguous; fp32 accumulation, RNE bf16 output.  Exact
 * lengths m*k, n*k, m*n.  Any m, n, k.  The pipelined 256x256 MFMA tile
 * (128x128 for small grids) runs whenever k is a multiple of 8 (k*512 <
 * 2^31) and A and B are 16-byte aligned, with a partial last k stage when k
 * is not a multiple of 64: whole tiles when m and n are multiples of 256
 * and C is 16-byte aligned, edge tiles (element-wise masked stores)
 * otherwise.  For other k or alignments, when m and n are at least 128, the
 * rows that cannot be read in place are first copied into aligned rows of
 * k rounded up to 8 (zeros past k) in stream-ordered scratch from the
 * library's pool and the tile runs on them (an operand that is only
 * misaligned gives the aligned operand's bits).  Smaller outputs, and
 * devices without a pool, take a bounds-checked 64x64-tile kernel; k = 0
 * writes +0. */
int32_t fe2o3_gemm_bf16_nt(const uint16_t *a, uint64_t a_len,
                           const uint16_t *b, uint64_t b_len, uint16_t *c,
                           uint64_t c_len, uint32_t m, uint32_t n, uint32_t k,
                           void *stream);

/* ---- row softmax ----------------------------------------------------------------- */

/* examples/row_softmax_v1/src/kernel.rs:13 row_softmax_v1(input: &[f32],
 * output: DisjointSlice<f32, GridExclusive>): one 64-element f32 row. */
int32_t fe2o3_row_softmax_v1(const float *input, uint64_t input_len,
                             float *output, uint64_t output_len, void *stream);

/* The same stable softmax over `rows` independent rows of `cols` f32 values
 * (max, sum of exp(x - max), divide; masked elements -> +0 as in
 * examples/row_softmax_v1/src/numerical_contract.rs:130-199).  mask may be
 * NULL (all active) or hold rows*cols bytes, nonzero = active.  A row with no
 * active element yields all +0.  Rejects cols == 0. */
int32_t fe2o3_row_softmax(const float *input, uint64_t input_len, float *output,
                          uint64_t output_len, const uint8_t *mask,
                          uint64_t mask_len, uint64_t rows, uint64_t cols,
                          void *stream);

/* ---- flash attention --------------------------------------------------------------- */

/* examples/flash_attention_v1/src/kernel.rs:130-135
 * flash_attention_causal_f32_b1_h1_n8_d16_v1(q, k, v: &[f32],
 * output: DisjointSlice<f32, Blocked<Index1D,1,2>>): causal, N=8, D=16,
 * scale 0.25 (examples/flash_attention_v1/src/contract.rs:3-31), f32. */
int32_t fe2o3_flash_attention_causal_f32_b1_h1_n8_d16_v1(
    const float *q, uint64_t q_len, const float *k, uint64_t k_len,
    const float *v, uint64_t v_len, float *output, uint64_t output_len,
    void *stream);

/* Flash-attention forward at the BASELINE shape: Q, K, V, O bf16
 * [batch, heads, seq, head_dim] (head_dim contiguous), O = softmax(scale *
 * Q K^T [+ causal mask]) V with fp32 online max/sum; lse (may be NULL)
 * receives the fp32 natural-log row statistic max + ln(sum) per
 * [batch, heads, seq].  head_dim must be 128 (FE2O3_ERR_SHAPE otherwise);
 * any seq >= 1 with seq * 256 < 2^31 (the last 128-row query tile and
 * 64-key tile of a head may be partial); scale positive and finite. */
int32_t fe2o3_flash_attention_fwd(const uint16_t *q, uint64_t q_len,
                                  const uint16_t *k, uint64_t k_len,
                                  const uint16_t *v, uint64_t v_len,
                                  uint16_t *o, uint64_t o_len, float *lse,
                                  uint64_t lse_len, uint32_t batch,
                                  uint32_t heads, uint32_t seq,
                                  uint32_t head_dim, int32_t causal,
                                  float scale, void *stream);

/* ---- top-2 MoE ------------------------------------------------------------------------ */

#define FE2O3_DROP_ROUTE 0xffffffffu

/* examples/moe_top2_v1/src/kernel.rs:102-111
 * moe_top2_route_f32_t8_e4_k2_c4_v1(logits: &[f32], top2_experts,
 * requested_counts, admitted_counts, expert_offsets, route_slots,
 * permutation, inverse_permutation: DisjointSlice<u32>): T=8, E=4,
 * capacity 4 (examples/moe_top2_v1/src/contract.rs:3-29).  Lengths 32, 16,
 * 4, 4, 5, 16, 16, 16. */
int32_t fe2o3_moe_top2_route_f32_t8_e4_k2_c4_v1(
    const float *logits, uint64_t logits_len, uint32_t *top2_experts,
    uint64_t top2_len, uint32_t *requested_counts, uint64_t requested_len,
    uint32_t *admitted_counts, uint64_t admitted_len, uint32_t *expert_offsets,
    uint64_t offsets_len, uint32_t *route_slots, uint64_t slots_len,
    uint32_t *permutation, uint64_t permutation_len, uint32_t *inverse,
    uint64_t inverse_len, void *stream);

/* The same router for any tokens x experts (experts in 2..64) and capacity
 * (FE2O3_DROP_ROUTE = unbounded): higher logit first, equal logits to the
 * lower expert id (kernel.rs:25-59); admitted = min(requested, capacity);
 * offsets = exclusive scan with terminal total; slots assigned to routes
 * (route = 2*token + rank) in route order; permutation/inverse with
 * FE2O3_DROP_ROUTE sentinels.  logits_dtype 0 = f32, 1 = bf16 bits.
 * route_weights (may be NULL): w0 = 1/(1+exp(l1-l0)), w1 = 1 - w0, so every
 * pair sums to exactly 1 (examples/moe_expert_v1/src/pipeline.rs:137-148).
 * Lengths: top2/slots/permutation/inverse/route_weights 2*tokens,
 * requested/admitted experts, offsets experts+1.  Above 8192 routes the
 * slot assignment takes 4 * (experts + 1) * (ceil(routes / 512) + 1) bytes
 * of stream-ordered scratch from the library's pool (the general GEMM's);
 * where the device has none, one kernel whose work grows as routes^2. */
int32_t fe2o3_moe_top2_route(const void *logits, uint64_t logits_len,
                             uint32_t logits_dtype, uint32_t *top2_experts,
                             uint64_t top2_len, uint32_t *requested_counts,
                             uint64_t requested_len, uint32_t *admitted_counts,
                             uint64_t admitted_len, uint32_t *expert_offsets,
                             uint64_t offsets_len, uint32_t *route_slots,
                             uint64_t slots_len, uint32_t *permutation,
                             uint64_t permutation_len, uint32_t *inverse,
                             uint64_t inverse_len, float *route_weights,
                             uint64_t weights_len, uint32_t tokens,
                             uint32_t experts, uint32_t capacity, void *stream);

/* examples/moe_expert_v1/src/kernel.rs:30-34
 * moe_expert_gemm_bf16_m16_n16_k16_v1(activations: &[u16], weights: &[u16],
 * output: DisjointSlice<f32, Blocked<Index1D,16,4>>): one 16x16x16 expert
 * tile, activations [16 rows, 16 hidden] and weights [16 hidden, 16 out]
 * row-major, output f32 [16,16].  Lengths 256. */
int32_t fe2o3_moe_expert_gemm_bf16_m16_n16_k16_v1(
    const uint16_t *activations, uint64_t activations_len,
    const uint16_t *weights, uint64_t weights_len, float *output,
    uint64_t output_len, void *stream);

/* examples/moe_expert_v1/src/kernel.rs:104-109
 * moe_expert_combine_f32_t8_k2_o16_v1(compact_output: &[f32], inverse: &[u32],
 * route_weights: &[f32], combined_output: DisjointSlice<f32>): T=8, K=2,
 * O=16; combined[t,o] = sum over ranks of w * compact[inverse[2t+rank], o]
 * in rank order from +0, dropped routes contribute nothing.  Lengths 256
 * (16 slots x 16), 16, 16, 128. */
int32_t fe2o3_moe_expert_combine_f32_t8_k2_o16_v1(
    const float *compact_output, uint64_t compact_len, const uint32_t *inverse,
    uint64_t inverse_len, const float *route_weights, uint64_t weights_len,
    float *combined_output, uint64_t combined_len, void *stream);

/* Scaled-up top-2 expert FFN (gate/up with SiLU, down), the BASELINE MoE
 * layer: for each admitted route r of token t to expert e,
 *   h = bf16( silu(x_t . Wg_e^T) * (x_t . Wu_e^T) ),  y_r = h . Wd_e^T,
 * and out[t] = bf16( sum over ranks of w_r * y_r ) (dropped routes add 0).
 * x [tokens, hidden] bf16; w_gate, w_up [experts, ffn, hidden] bf16;
 * w_down [experts, hidden, ffn] bf16; routing arrays as produced by
 * fe2o3_moe_top2_route; out [tokens, hidden] bf16.  hidden must be a
 * multiple of 256 and ffn a multiple of 128.  workspace: device scratch of
 * at least fe2o3_moe_ffn_workspace_bytes(tokens, hidden, ffn, experts)
 * bytes.  The routing arrays are device data the host cannot validate: a
 * routing that fails fe2o3_moe_routing_check gives unspecified outputs, but
 * every access stays inside the caller's buffers and the workspace (offsets
 * are clamped to [0, 2*tokens]; slot and permutation entries out of range
 * count as dropped). */
uint64_t fe2o3_moe_ffn_workspace_bytes(uint32_t tokens, uint32_t hidden,
                                       uint32_t ffn, uint32_t experts);
int32_t fe2o3_moe_ffn_top2(const uint16_t *x, uint64_t x_len,
                           const uint16_t *w_gate, uint64_t w_gate_len,
                           const uint16_t *w_up, uint64_t w_up_len,
                           const uint16_t *w_down, uint64_t w_down_len,
                           const uint32_t *top2_experts, uint64_t top2_len,
                           const uint32_t *expert_offsets, uint64_t offsets_len,
                           const uint32_t *permutation, uint64_t permutation_len,
                           const uint32_t *inverse, uint64_t inverse_len,
                           const float *route_weights, uint64_t weights_len,
                           uint16_t *out, uint64_t out_len, void *workspace,
                           uint64_t workspace_bytes, uint32_t tokens,
                           uint32_t hidden, uint32_t ffn, uint32_t experts,
                           void *stream);

/* Allocation-free variant of fe2o3_moe_ffn_top2.  It has no counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as fe2o3_moe_ffn_top2 without the
 * workspace: the scratch is a library-owned device array of 64 MiB per GPU
 * (FE2O3_MOE_NOALLOC_SCRATCH_BYTES), held from library load to process end,
 * so fe2o3_moe_ffn_workspace_bytes(tokens, hidden, ffn, experts) must not
 * exceed it (else FE2O3_ERR_WORKSPACE; e.g. up to 481 tokens at hidden 4096,
 * ffn 14336).  The call launches every kernel on `stream` and allocates or
 * creates nothing (no memory, stream or event).  Every call on a GPU shares
 * that GPU's scratch, so calls that overlap on one GPU (different streams,
 * or host threads) race and must be serialized by the caller; no part of
 * the scratch needs to start at zero (each call writes every row it reads). */
#define FE2O3_MOE_NOALLOC_SCRATCH_BYTES (UINT64_C(64) << 20)
int32_t fe2o3_moe_ffn_top2_noalloc(
    const uint16_t *x, uint64_t x_len, const uint16_t *w_gate, uint64_t w_gate_len,
    const uint16_t *w_up, uint64_t w_up_len, const uint16_t *w_down,
    uint64_t w_down_len, const uint32_t *top2_experts, uint64_t top2_len,
    const uint32_t *expert_offsets, uint64_t offsets_len,
    const uint32_t *permutation, uint64_t permutation_len,
    const uint32_t *inverse, uint64_t inverse_len, const float *route_weights,
    uint64_t weights_len, uint16_t *out, uint64_t out_len, uint32_t tokens,
    uint32_t hidden, uint32_t ffn, uint32_t experts, void *stream);

/* ---- gfx942 FNUZ fp8 values ----------------------------------------------------------
 * crates/fe2o3-device/src/fp8.rs:85-95 and :193-203 (Fp8E4M3Fnuz / Fp8E5M2Fnuz
 * ::from_f32 and ::to_f32; bodies f32_to_fnuz / fnuz_to_f32, :296-381), over
 * whole device arrays.  FNUZ: one unsigned zero 0x00, sole NaN 0x80, no
 * infinities.  E4M3 FNUZ: bias 8, finite range +-240; E5M2 FNUZ: bias 16,
 * +-57344.  The reference's packed Fp8*Fnuzx4 (fp8.rs:272-294, 435-518; lane i in bits
 * 8i..8i+7) is the little-endian 32-bit view of four consecutive codes. */
#define FE2O3_FP8_FNUZ_E4M3 0
#define FE2O3_FP8_FNUZ_E5M2 1

/* q[i] = from_f32(x[i]): round to nearest, ties to even; a magnitude above
 * the largest finite value saturates to it; NaN and +-inf give 0x80;
 * whatever rounds to zero (negative zero included) gives 0x00.  Any
 * alignment (16-byte accesses when x and q are both 16-byte aligned).
 * FE2O3_ERR_SHAPE for another format, FE2O3_ERR_LENGTH when the lengths
 * differ; n = 0 launches nothing. */
int32_t fe2o3_fp8_fnuz_from_f32(const float *x, uint64_t x_len, uint8_t *q,
                                uint64_t q_len, int32_t format, void *stream);
/* x[i] = to_f32(q[i]), exact; 0x80 gives the f32 bits 0xffc00000 (the
 * negative quiet NaN gfx942 widens it to).  Errors as above. */
int32_t fe2o3_fp8_fnuz_to_f32(const uint8_t *q, uint64_t q_len, float *x,
                              uint64_t x_len, int32_t format, void *stream);

/* crates/fe2o3-device/src/half.rs:182-190 (Bf16::from_f32) over an array:
 * out[i] = the bf16 bits of x[i], round to nearest, ties to even; a NaN
 * keeps its sign and high payload bits and is quieted (| 0x0040).  The
 * narrowing every bf16 output of the library goes through (gfx950's
 * v_cvt_pk_bf16_f32).  Any alignment (16-byte loads and 8-byte stores when
 * x is 16-byte and out 8-byte aligned).  FE2O3_ERR_LENGTH when the lengths
 * differ; n = 0 launches nothing. */
int32_t fe2o3_bf16_from_f32(const float *x, uint64_t x_len, uint16_t *out,
                            uint64_t out_len, void *stream);

/* ---- fp8 (OCP E4M3FN, per-tensor scale) ---------------------------------------------
 * Not in the reference (its only fp8 type is gfx942 FNUZ,
 * crates/fe2o3-device/src/fp8.rs:53-110, which gfx950's MFMA does not take):
 * the quantized-inference path of the BASELINE configuration. */

/* amax[0] = max |x[i]| (NaN-free input assumed; 0 for n == 0). */
int32_t fe2o3_amax_f32(const float *x, uint64_t x_len, float *amax, void *stream);
/* scale[0] = max(amax[0], tiny) / 448 (device to device). */
int32_t fe2o3_fp8_scale_from_amax(const float *amax, float *scale, void *stream);
/* q[i] = e4m3_satfinite_rne(x[i] / scale[0]) (one correctly rounded f32
 * division per element). */
int32_t fe2o3_quantize_e4m3(const float *x, uint64_t x_len, const float *scale,
                            uint8_t *q, uint64_t q_len, void *stream);
/* C[m,n] bf16 = (scale_a[0]*scale_b[0]) * (A_q[m,k] . B_q[n,k]^T), fp32
 * accumulation; A row-major, B stored [n,k] (k contiguous).  Any m, n, k.
 * The pipelined fp8 MFMA tile runs whenever k is a multiple of 16
 * (k*256 < 2^31; a partial last stage when k is not a multiple of 128) and
 * A and B are 16-byte aligned (edge tiles for m or n not a multiple of 256
 * or an unaligned C).  For other k or alignments, when m and n are at least
 * 128, the rows that cannot be read in place are first copied into aligned
 * rows of k rounded up to 16 (E4M3 +0 past k) in stream-ordered scratch
 * from the library's pool and the tile runs on them; smaller outputs, and
 * devices without a pool, take a bounds-checked kernel that widens E4M3 to
 * bf16 exactly and multiplies on bf16 MFMAs.  k = 0 writes +0.  The
 * products of two E4M3 values are exact in fp32 on every path. */
int32_t fe2o3_gemm_fp8_nt(const uint8_t *a, uint64_t a_len, const uint8_t *b,
                          uint64_t b_len, const float *scale_a,
                          const float *scale_b, uint16_t *c, uint64_t c_len,
                          uint32_t m, uint32_t n, uint32_t k, void *stream);

/* crates/fe2o3-host/src/moe_routing_expert_bridge_v1.rs:220-389
 * (check_host_observed_moe_routing_output_v1) with the compact pack plan of
 * crates/fe2o3-host/src/generated_moe_expert_v1.rs:159-190, on the device
 * and for any tokens (2 * tokens below 2^32), experts (1..64) and capacity
 * (0xFFFFFFFF = unbounded).  Above 1024 tokens the check runs over
 * workgroups of 256 tokens on stream-ordered scratch from the library's
 * pool (about 4 * (2 * tokens + (2 * tokens / 512 + 1) * (experts + 7))
 * bytes); where the device has no pool, one workgroup up to 12288 tokens,
 * and above that the allocation's HIP error.  Checks a complete routing
 * output (the seven arrays of fe2o3_moe_top2_route) and writes the reference's FIRST failing
 * relation to record[0..3] = {kind, index, expected, actual}, kind
 * FE2O3_RC_OK (0) when every relation holds.  Lengths as
 * fe2o3_moe_top2_route; record 4. */
enum {
  FE2O3_RC_OK = 0,
  FE2O3_RC_EXPERT_OUT_OF_RANGE = 1,    /* index route, actual expert            */
  FE2O3_RC_DUPLICATE_TOKEN_EXPERT = 2, /* index token, actual expert            */
  FE2O3_RC_REQUESTED_COUNT = 3,        /* index expert, expected, actual        */
  FE2O3_RC_CAPACITY = 4,               /* index expert, actual admitted         */
  FE2O3_RC_ADMITTED_COUNT = 5,         /* index expert, expected, actual        */
  FE2O3_RC_FIRST_OFFSET = 6,           /* actual offsets[0]                     */
  FE2O3_RC_NONMONOTONE_OFFSETS = 7,    /* index expert, expected start, actual end */
  FE2O3_RC_OFFSET_MISMATCH = 8,        /* index expert + 1, expected, actual    */
  FE2O3_RC_PLAN_OFFSET_ORDER = 9,      /* index expert, actual end              */
  FE2O3_RC_PLAN_CAPACITY = 10,         /* index expert, actual rows             */
  FE2O3_RC_SLOT_OUT_OF_RANGE = 11,     /* index route, expected accepted, actual slot */
  FE2O3_RC_DUPLICATE_SLOT = 12,        /* index route, actual slot              */
  FE2O3_RC_STABLE_SLOT = 13,           /* index route, expected, actual         */
  FE2O3_RC_INVERSE = 14,               /* index route, expected, actual         */
  FE2O3_RC_PERMUTATION = 15,           /* index slot, expected route, actual    */
  FE2O3_RC_PREFIX_HOLE = 16,           /* index slot                            */
  FE2O3_RC_PERMUTATION_ROUTE = 17,     /* index slot, actual route              */
  FE2O3_RC_PERMUTATION_TAIL = 18       /* index slot, actual                    */
};
int32_t fe2o3_moe_routing_check(const uint32_t *top2_experts, uint64_t top2_len,
                                const uint32_t *requested_counts, uint64_t requested_len,
                                const uint32_t *admitted_counts, uint64_t admitted_len,
                                const uint32_t *expert_offsets, uint64_t offsets_len,
                                const uint32_t *route_slots, uint64_t slots_len,
                                const uint32_t *permutation, uint64_t permutation_len,
                                const uint32_t *inverse, uint64_t inverse_len,
                                uint32_t tokens, uint32_t experts, uint32_t capacity,
                                uint32_t *record, uint64_t record_len, void *stream);

/* ---- kernel resource observation ------------------------------------------------------- */

/* crates/fe2o3-host/src/generated_lds_gemm_lifecycle.rs:47-120
 * (ExactLdsGemmKernelResourceObservationV1: group and private segment
 * sizes observed from the loaded code object).  Kernel `index` of those
 * that C-ABI entry point `entry` launches: its workgroup size and dynamic
 * LDS (launch facts), its static LDS (group segment), private segment
 * bytes per lane (0 = no scratch, no register spills) and registers as the
 * runtime reports them for the loaded code object.  *count is always set
 * to the number of kernels behind `entry`; FE2O3_ERR_LENGTH when
 * index >= *count (0 for an unknown entry); FE2O3_ERR_OVERFLOW (and
 * *count 0) if the library's kernel table overflowed when it loaded.
 * 120-byte record. */
typedef struct Fe2o3KernelResources {
  char kernel[96];
  uint32_t workgroup_size;
  uint32_t static_lds_bytes;
  uint32_t dynamic_lds_bytes;
  uint32_t private_segment_bytes;
  uint32_t vgprs;
  uint32_t max_threads_per_workgroup;
} Fe2o3KernelResources;
int32_t fe2o3_kernel_resources(const char *entry, uint32_t index, Fe2o3KernelResources *out,
                               uint32_t *count);

/* ---- typed lifecycle of the exact LDS GEMM code object -----------------------------------
 *
 * crates/fe2o3-host/src/generated_lds_gemm_lifecycle.rs: a one-shot,
 * linear lifecycle over one code object of the exact 16x16x16 LDS GEMM
 * profile: join (:276) -> load (:298) -> dispatch_and_wait (:391) ->
 * unload (:522).  The code object is the library's own gfx950 build of
 * tiled_gemm_lds_v1 (code object v6, xnack-), embedded in the library; it
 * is never exposed.  Its kernarg ABI is the reference's: 48 explicit bytes
 * ({u64 address, u64 elements} for A, B and C), then a 256-byte implicit
 * suffix initialized for the launch geometry, 304 bytes in all, 8-byte
 * aligned in the descriptor and 16-byte aligned for the dispatch.
 *
 * The lifecycle is an opaque handle whose state only moves forward:
 *   JOINED --load--> LOADED --dispatch_and_wait--> COMPLETED --unload--> (receipt, freed)
 * A failed load or dispatch performs every cleanup the reached state needs
 * (kernel dropped, then one terminal unload, then the A/B/C leases and the
 * adapter released) and leaves the handle FAILED.  Calling a transition in
 * another state returns FE2O3_ERR_STATE and changes nothing.
 * fe2o3_lds_gemm_slice1_release_v1 frees a handle in any state, unloading
 * first when it holds a loaded executable (the reference's Drop).  An
 * unload that the adapter reports as failed, or whose observation does not
 * match the load, aborts the process (generated_lds_gemm_lifecycle.rs:
 * 779-806): the executable's state is then unknown.
 *
 * Runtime access goes through an adapter: a table of callbacks
 * (ReviewedExactLdsGemmRuntimeAdapterV1, :101-121, and the HSA lifecycle
 * adapter it extends).  fe2o3_lds_gemm_slice1_hip_adapter_v1 returns the
 * library's HIP adapter (module load from memory, function resolution,
 * resource query, module launch with an explicit kernarg buffer, stream
 * synchronize, module unload).  A caller may supply its own table, e.g.
 * to observe or fault-inject the lifecycle without a GPU.  Adapter
 * callbacks return 0 on success, anything else on failure; the lifecycle
 * validates every observation they return against what it asked for.
 */
#define FE2O3_ERR_JOIN (-27)     /* code object / host request reconciliation failed */
#define FE2O3_ERR_LOAD (-28)     /* environment, load, resolution or resources rejected */
#define FE2O3_ERR_DISPATCH (-29) /* implicit kernarg or dispatch rejected                */
#define FE2O3_ERR_STATE (-30)    /* lifecycle call out of order                         */

#define FE2O3_SLICE1_EXPLICIT_KERNARG_BYTES 48u
#define FE2O3_SLICE1_IMPLICIT_KERNARG_BYTES 256u
#define FE2O3_SLICE1_COMPLETE_KERNARG_BYTES 304u
#define FE2O3_SLICE1_CONTRACT_KERNARG_ALIGNMENT 8u
#define FE2O3_SLICE1_HSA_KERNARG_ALIGNMENT 16u
#define FE2O3_SLICE1_STATIC_LDS_BYTES 1024u

/* lifecycle states */
enum {
  FE2O3_SLICE1_JOINED = 1,
  FE2O3_SLICE1_LOADED = 2,
  FE2O3_SLICE1_COMPLETED = 3,
  FE2O3_SLICE1_FAILED = 4
};

/* error kinds: ExactLdsGemmSlice1JoinErrorV1 (:126-135), the host-request
 * preparation errors of crates/fe2o3-host/src/generated_lds_gemm.rs:676-720,
 * ExactLdsGemmSlice1LoadErrorV1 (:167-177) and
 * ExactLdsGemmSlice1DispatchErrorV1 (:216-223). */
enum {
  FE2O3_SLICE1_E_NONE = 0,
  FE2O3_SLICE1_E_IMPORT_IDENTITY = 1,
  FE2O3_SLICE1_E_PROFILE_IDENTITY = 2,
  FE2O3_SLICE1_E_CONTRACT = 3,
  FE2O3_SLICE1_E_FINALIZED_OUTPUT = 4,  /* field: which code-object fact drifted */
  FE2O3_SLICE1_E_CONTRACT_FIELD = 5,
  FE2O3_SLICE1_E_BUFFER_CONTRACT = 6,   /* index: buffer                          */
  FE2O3_SLICE1_E_HOST_LENGTH_IDENTITY = 7,
  FE2O3_SLICE1_E_HOST_FIELD = 8,
  FE2O3_SLICE1_E_HOST_LENGTH = 9,       /* index: role, expected, actual          */
  FE2O3_SLICE1_E_HOST_NULL = 10,
  FE2O3_SLICE1_E_HOST_ALIGNMENT = 11,   /* expected: required bytes               */
  FE2O3_SLICE1_E_HOST_OUTPUT_OVERLAP = 12, /* index: the input C overlaps         */
  FE2O3_SLICE1_E_HOST_ADDRESS_OVERFLOW = 13,
  FE2O3_SLICE1_E_RECEIPT_FIELD = 14,    /* protected profiles: field names it  */
  FE2O3_SLICE1_E_CONTEXT_IDENTITY = 20,
  FE2O3_SLICE1_E_ENVIRONMENT_ADAPTER = 21,
  FE2O3_SLICE1_E_ENVIRONMENT = 22,
  FE2O3_SLICE1_E_LOAD_ADAPTER = 23,
  FE2O3_SLICE1_E_LOAD_OBSERVATION = 24,
  FE2O3_SLICE1_E_KERNEL_ADAPTER = 25,
  FE2O3_SLICE1_E_KERNEL_OBSERVATION = 26,
  FE2O3_SLICE1_E_RESOURCE_ADAPTER = 27,
  FE2O3_SLICE1_E_RESOURCE_OBSERVATION = 28,
  FE2O3_SLICE1_E_IMPLICIT_ADAPTER = 40,
  FE2O3_SLICE1_E_IMPLICIT_OBSERVATION = 41,
  FE2O3_SLICE1_E_EXPLICIT_KERNARG_MUTATION = 42,
  FE2O3_SLICE1_E_DISPATCH_ADAPTER = 43,
  FE2O3_SLICE1_E_DISPATCH_OBSERVATION = 44
};

typedef struct Fe2o3Slice1ErrorV1 {
  int32_t kind;           /* FE2O3_SLICE1_E_*                                 */
  int32_t index;          /* buffer / role index where the kind names one, else -1 */
  int32_t adapter_status; /* what the failing adapter callback returned, else 0 */
  int32_t reserved;
  uint64_t expected, actual;
  char field[64];         /* the drifted field, as the reference names it, or "" */
} Fe2o3Slice1ErrorV1;

/* roles 1 = A, 2 = B, 3 = C; element 1 = bf16 bits in u16, 2 = f32;
 * ownership 0 = shared borrow, 1 = unique borrow; access 0 = read-only,
 * 1 = read-write; alias 0 = shared read-only, 1 = exclusive. */
typedef struct Fe2o3Slice1BufferContractV1 {
  uint32_t role, element;
  uint64_t elements, bytes;
  uint8_t length_identity[32];
  uint32_t ownership, access, alias, reserved;
} Fe2o3Slice1BufferContractV1;

/* ExactLdsGemmContractV1 (crates/fe2o3-hsaco-finalize/src/
 * lds_gemm_profile_registry.rs:606-670) for the gfx950 code object. */
typedef struct Fe2o3Slice1ContractV1 {
  uint32_t profile;  /* 1 = Slice1M16N16K16 */
  uint32_t code_object_version;
  char target[32];
  uint8_t identity[32];
  uint32_t grid[3], workgroup[3];
  uint32_t wavefront_size;
  uint32_t explicit_kernarg_bytes, complete_kernarg_bytes, kernarg_alignment;
  uint32_t static_lds_bytes, lds_allocations, lds_bytes_per_allocation, lds_alignment;
  Fe2o3Slice1BufferContractV1 buffers[3];
} Fe2o3Slice1ContractV1;

/* What the embedded code object itself says: ELF header, kernel descriptor
 * (tiled_gemm_lds_v1.kd) and the AMDGPU metadata note. */
typedef struct Fe2o3Slice1InspectionV1 {
  uint64_t byte_len;
  uint32_t code_object_version; /* from EI_ABIVERSION                              */
  uint32_t e_flags;
  char target[64];              /* metadata amdhsa.target, without the triple      */
  uint32_t kd_group_segment_bytes, kd_private_segment_bytes, kd_kernarg_bytes, kd_wavefront_size;
  uint32_t md_kernarg_bytes, md_kernarg_alignment, md_group_segment_bytes,
      md_private_segment_bytes;
  uint32_t md_wavefront_size, md_max_flat_workgroup_size;
  uint32_t explicit_args, explicit_bytes; /* by-value arguments and their extent   */
  uint32_t implicit_offset, implicit_bytes; /* first hidden argument, suffix bytes */
  uint32_t sgpr_spills, vgpr_spills, uses_dynamic_stack, reserved;
} Fe2o3Slice1InspectionV1;

/* The finalized artifact: identities, contract and inspection.  The
 * finalizer identity is the SHA-256 of the code-object bytes computed now;
 * build_digest is the SHA-256 recorded when the library was built. */
typedef struct Fe2o3Slice1ArtifactV1 {
  uint8_t finalizer_identity[32];
  uint8_t build_digest[32];
  uint8_t import_identity[32];
  uint8_t profile_identity[32];
  Fe2o3Slice1ContractV1 contract;
  Fe2o3Slice1InspectionV1 inspection;
} Fe2o3Slice1ArtifactV1;

/* JoinFactsV1 (:985-1034): everything join reconciles, as booleans for the
 * identity comparisons plus the contract and host-request fields.
 * inspection_matches: the code object's own ELF/descriptor/metadata facts
 * agree with the contract (checked with finalized_output_matches). */
typedef struct Fe2o3Slice1JoinFactsV1 {
  uint8_t import_matches, profile_matches, contract_matches, finalized_output_matches;
  uint8_t inspection_matches, host_profile_identity_matches, reserved[2];
  Fe2o3Slice1ContractV1 contract;
  char host_target[32];
  uint32_t host_profile;
  uint32_t host_grid[3], host_workgroup[3];
  uint32_t host_static_lds, host_dynamic_lds;
  uint32_t host_explicit_kernarg, host_complete_kernarg, host_kernarg_alignment;
  uint8_t host_length_identities[3][32];
} Fe2o3Slice1JoinFactsV1;

typedef struct Fe2o3Slice1GeometryV1 {
  uint32_t grid[3], workgroup[3], dynamic_lds_bytes;
} Fe2o3Slice1GeometryV1;

/* Observations (crates/fe2o3-host/src/hsa_executable_lifecycle.rs types of
 * the same names).  Object identities are 16 opaque bytes. */
typedef struct Fe2o3Slice1EnvironmentV1 {
  uint8_t runtime_instance[16];
  char physical_target[64];
  int32_t hip_ordinal;
  uint8_t physical_uuid[16];
  char agent_target[64];
  uint64_t agent_handle;
  uint8_t agent_runtime_instance[16];
  uint8_t agent_physical_uuid[16];
} Fe2o3Slice1EnvironmentV1;

typedef struct Fe2o3Slice1LoadV1 {
  uint8_t digest[32];
  uint64_t byte_len;
  uint8_t runtime_instance[16];
  uint64_t agent_handle;
  uint8_t executable_object[16];
} Fe2o3Slice1LoadV1;

typedef struct Fe2o3Slice1ResolutionV1 {
  uint8_t executable_object[16], kernel_object[16];
  char symbol[64];
  uint64_t kernarg_segment_bytes, kernarg_alignment;
} Fe2o3Slice1ResolutionV1;

typedef struct Fe2o3Slice1ResourcesV1 {
  uint8_t executable_object[16], kernel_object[16];
  uint32_t group_segment_bytes, private_segment_bytes;
} Fe2o3Slice1ResourcesV1;

typedef struct Fe2o3Slice1ImplicitV1 {
  uint8_t executable_object[16], kernel_object[16];
  Fe2o3Slice1GeometryV1 geometry;
  uint64_t explicit_bytes, implicit_offset, implicit_bytes;
  uint32_t completed, reserved;
} Fe2o3Slice1ImplicitV1;

typedef struct Fe2o3Slice1DispatchV1 {
  uint8_t dispatch_identity[16];
  uint8_t executable_object[16], kernel_object[16];
  Fe2o3Slice1GeometryV1 geometry;
  uint32_t completed;
} Fe2o3Slice1DispatchV1;

typedef struct Fe2o3Slice1UnloadV1 {
  uint8_t executable_object[16];
  uint8_t runtime_instance[16];
  uint64_t agent_handle;
  uint32_t released, reserved;
} Fe2o3Slice1UnloadV1;

/* The runtime adapter.  `self` is passed back to every callback.  The
 * lifecycle takes the table over at load and calls drop_adapter exactly
 * once when it is done with it (also when load fails).  Handles
 * (`executable`, `kernel`) are the adapter's own opaque values. */
typedef struct Fe2o3Slice1AdapterV1 {
  void *self;
  int32_t (*context_identity)(void *self, uint8_t identity[16]);
  int32_t (*observe_environment)(void *self, Fe2o3Slice1EnvironmentV1 *out);
  int32_t (*load_executable)(void *self, const uint8_t *bytes, uint64_t byte_len,
                             const uint8_t digest[32], uint64_t *executable,
                             Fe2o3Slice1LoadV1 *out);
  int32_t (*resolve_kernel)(void *self, uint64_t executable, const char *symbol,
                            uint64_t *kernel, Fe2o3Slice1ResolutionV1 *out);
  int32_t (*observe_resources)(void *self, uint64_t executable, uint64_t kernel,
                               Fe2o3Slice1ResourcesV1 *out);
  int32_t (*initialize_implicit_kernarg)(void *self, uint64_t executable, uint64_t kernel,
                                         const Fe2o3Slice1GeometryV1 *geometry,
                                         uint64_t explicit_bytes, uint64_t implicit_offset,
                                         uint64_t implicit_bytes, uint8_t *kernarg,
                                         uint64_t kernarg_bytes, Fe2o3Slice1ImplicitV1 *out);
  int32_t (*launch_and_wait)(void *self, uint64_t executable, uint64_t kernel,
                             const Fe2o3Slice1GeometryV1 *geometry, uint8_t *kernarg,
                             uint64_t kernarg_bytes, Fe2o3Slice1DispatchV1 *out);
  void (*drop_kernel)(void *self, uint64_t kernel);
  int32_t (*unload_executable)(void *self, uint64_t executable, Fe2o3Slice1UnloadV1 *out);
  void (*drop_adapter)(void *self);
} Fe2o3Slice1AdapterV1;

/* Terminal receipt (UnloadedExactLdsGemmSlice1V1, :569-607). */
typedef struct Fe2o3Slice1ReceiptV1 {
  uint8_t finalizer_identity[32], import_identity[32], profile_identity[32];
  uint8_t executable_object[16], kernel_object[16], dispatch_identity[16];
  uint8_t unload_identity[32];
} Fe2o3Slice1ReceiptV1;

/* Descriptive view of a live handle. */
typedef struct Fe2o3Slice1ObservationV1 {
  int32_t state;
  uint32_t leases_retained; /* the handle still refers to A, B and C */
  uint32_t holds_executable, holds_kernel;
  Fe2o3Slice1EnvironmentV1 environment;
  Fe2o3Slice1LoadV1 load;
  Fe2o3Slice1ResolutionV1 resolution;
  Fe2o3Slice1ResourcesV1 resources;
  uint8_t dispatch_identity[16];
  Fe2o3Slice1ErrorV1 last_error;
} Fe2o3Slice1ObservationV1;

typedef struct Fe2o3Slice1Lifecycle Fe2o3Slice1Lifecycle;

/* The embedded artifact's identities, contract and inspection. */
int32_t fe2o3_lds_gemm_slice1_artifact_v1(Fe2o3Slice1ArtifactV1 *out);
/* JoinFactsV1::from_exact for the embedded artifact and the canonical host
 * request, and validate_join over any facts (:1036-1094, :1168-1218): the first
 * mismatch in the reference's order, as FE2O3_ERR_JOIN plus *error. */
int32_t fe2o3_lds_gemm_slice1_join_facts_v1(Fe2o3Slice1JoinFactsV1 *out);
int32_t fe2o3_lds_gemm_slice1_validate_join_v1(const Fe2o3Slice1JoinFactsV1 *facts,
                                               Fe2o3Slice1ErrorV1 *error);
/* Prepare the host request (A, B: 256 bf16 values, 2-byte aligned; C: 256
 * f32, 4-byte aligned and disjoint from A and B; generated_lds_gemm.rs:
 * 559-670) and join it to the embedded artifact.  `release_leases`, if
 * given, is called with `user` exactly once, when the handle stops
 * referring to A, B and C (at completion, failure or release).  `device`
 * is the HIP ordinal the buffers belong to; load checks the adapter's
 * context identity against it. */
int32_t fe2o3_lds_gemm_slice1_join_v1(const uint16_t *a, uint64_t a_len, const uint16_t *b,
                                      uint64_t b_len, float *c, uint64_t c_len, int32_t device,
                                      void (*release_leases)(void *user), void *user,
                                      Fe2o3Slice1Lifecycle **out, Fe2o3Slice1ErrorV1 *error);
/* The library's HIP adapter bound to `device` (context identity: the
 * ordinal and this process). */
int32_t fe2o3_lds_gemm_slice1_hip_adapter_v1(int32_t device, Fe2o3Slice1AdapterV1 *out);
/* The context identity a handle joined for `device` expects. */
int32_t fe2o3_lds_gemm_slice1_context_identity_v1(int32_t device, uint8_t identity[16]);
int32_t fe2o3_lds_gemm_slice1_load_v1(Fe2o3Slice1Lifecycle *lifecycle,
                                      const Fe2o3Slice1AdapterV1 *adapter,
                                      Fe2o3Slice1ErrorV1 *error);
int32_t fe2o3_lds_gemm_slice1_dispatch_and_wait_v1(Fe2o3Slice1Lifecycle *lifecycle,
                                                   Fe2o3Slice1ErrorV1 *error);
/* COMPLETED only: terminal unload, receipt, handle freed. */
int32_t fe2o3_lds_gemm_slice1_unload_v1(Fe2o3Slice1Lifecycle *lifecycle,
                                        Fe2o3Slice1ReceiptV1 *receipt);
void fe2o3_lds_gemm_slice1_release_v1(Fe2o3Slice1Lifecycle *lifecycle);
int32_t fe2o3_lds_gemm_slice1_observe_v1(const Fe2o3Slice1Lifecycle *lifecycle,
                                         Fe2o3Slice1ObservationV1 *out);
/* SHA-256 (FIPS 180-4), the digest every identity above is built from. */
int32_t fe2o3_sha256_v1(const void *data, uint64_t len, uint8_t digest[32]);

/* ---- protected profile lifecycles ------------------------------------------------------
 *
 * The same one-shot lifecycle for three more exact profiles, each over its
 * own gfx950 code object (code object v6, xnack-) built from
 * fe2o3_amd/csrc/codeobj/<name>.hip and embedded in the library:
 *   FE2O3_PROFILE_FLASH_ATTENTION_V1 (crates/fe2o3-host/src/
 *     flash_attention_v1_lifecycle.rs): flash_attention_causal_f32_b1_h1_n8_d16_v1,
 *     regions Q, K, V (read) and output (written), 128 f32 each; 64 explicit
 *     kernarg bytes, 320 in all.
 *   FE2O3_PROFILE_ROW_SOFTMAX_V1 (protected_row_softmax_v1_lifecycle.rs):
 *     row_softmax_v1, regions input (read) and output (written), 64 f32
 *     each; 32 / 288 bytes.
 *   FE2O3_PROFILE_MOE_TOP2_V1 (moe_top2_v1_lifecycle.rs):
 *     moe_top2_route_f32_t8_e4_k2_c4_v1, regions logits (read, 32 f32), then
 *     top2 (16), requested (4), admitted (4), offsets (5), slots (16),
 *     permutation (16) and inverse (16) u32 (written); 128 / 384 bytes.
 * Every profile launches grid [1,1,1] x workgroup [64,1,1] with no LDS and
 * no private segment, its explicit kernarg one {u64 address, u64 elements}
 * per region in role order.
 *
 * The handle, its states and transitions, the runtime adapter table and its
 * observations, the error record and the abort on an ambiguous unload are
 * the LDS GEMM lifecycle's above (an Fe2o3ProtectedLifecycleV1 is that
 * handle bound to another code object): join -> load -> dispatch_and_wait
 * -> unload, each failure doing the cleanup its state owes.
 *
 * Join runs the reference's order: the host request's regions (each region
 * in role order: its length, a non-null address, element alignment, no
 * address overflow; then every pair of regions that includes a written one
 * must not overlap -- read-only inputs may alias), then validate_join: the
 * profile's receipt fields (FE2O3_SLICE1_E_RECEIPT_FIELD, field = the
 * reference's name) and its host fields (FE2O3_SLICE1_E_HOST_FIELD), each
 * list in the reference's order.  The receipt fields are facts of the
 * embedded artifact as this library checks them: the identities are
 * nonzero, the code object's own ELF/descriptor/metadata facts (target, code
 * object version, kernarg sizes, segment sizes, spill counts) agree with the
 * profile, and the bytes are the ones the build recorded. */
#define FE2O3_PROTECTED_MAX_COMPLETE_KERNARG_BYTES 384u
#define FE2O3_PROTECTED_MAX_REGIONS 8u

enum {
  FE2O3_PROFILE_FLASH_ATTENTION_V1 = 1,
  FE2O3_PROFILE_ROW_SOFTMAX_V1 = 2,
  FE2O3_PROFILE_MOE_TOP2_V1 = 3
};

typedef struct Fe2o3ProtectedRegionV1 {
  const void *address;
  uint64_t elements;
} Fe2o3ProtectedRegionV1;

/* The profile's fixed facts. */
typedef struct Fe2o3ProtectedProfileV1 {
  uint32_t profile;
  uint32_t code_object_version;
  char name[32];
  char target[32];
  char symbol[64];
  uint32_t grid[3], workgroup[3];
  uint32_t dynamic_lds_bytes, static_lds_bytes, private_segment_bytes;
  uint32_t explicit_kernarg_bytes, complete_kernarg_bytes, kernarg_alignment;
  uint32_t hsa_kernarg_alignment;
  uint32_t regions;
  uint64_t region_elements[FE2O3_PROTECTED_MAX_REGIONS];
  uint32_t region_element_bytes[FE2O3_PROTECTED_MAX_REGIONS];
  uint32_t region_writes[FE2O3_PROTECTED_MAX_REGIONS];
  uint32_t shape[4]; /* flash B, H, N, D; softmax row elements; MoE T, E, K, C */
  uint32_t receipt_fields, host_fields;
  char receipt_field[16][40]; /* validate_join's receipt checks, in order */
  char host_field[16][40];    /* and its host checks */
} Fe2o3ProtectedProfileV1;

/* The embedded artifact.  artifact_identity: SHA-256 of the code-object
 * bytes now; build_digest: recorded when the library was built;
 * source_digest: of the kernel source; compiler_identity: over the compiler
 * version and flags; profile_identity: over the profile's facts; identity:
 * the receipt identity over all of these. */
typedef struct Fe2o3ProtectedArtifactV1 {
  uint8_t identity[32];
  uint8_t profile_identity[32];
  uint8_t artifact_identity[32];
  uint8_t build_digest[32];
  uint8_t source_digest[32];
  uint8_t compiler_identity[32];
  Fe2o3Slice1InspectionV1 inspection;
  Fe2o3ProtectedProfileV1 profile;
} Fe2o3ProtectedArtifactV1;

/* Everything validate_join reconciles: the receipt checks as booleans (in
 * the profile's receipt_field order) and the host request's fields. */
typedef struct Fe2o3ProtectedJoinFactsV1 {
  uint32_t profile;
  uint8_t receipt[16];
  char host_target[32];
  uint32_t host_shape[4];
  uint64_t host_argument_elements; /* flash: elements per region */
  uint32_t host_grid[3], host_workgroup[3];
  uint32_t host_code_object_version;
  uint32_t host_explicit_kernarg, host_complete_kernarg, host_kernarg_alignment;
  uint32_t host_policy; /* 1: causal / unmasked all-64 / routing-only, as the profile names */
} Fe2o3ProtectedJoinFactsV1;

typedef struct Fe2o3ProtectedReceiptV1 {
  uint8_t identity[32], artifact_identity[32];
  uint8_t executable_object[16], kernel_object[16], dispatch_identity[16];
  uint8_t unload_identity[32];
} Fe2o3ProtectedReceiptV1;

typedef struct Fe2o3Slice1Lifecycle Fe2o3ProtectedLifecycleV1;

int32_t fe2o3_protected_profile_v1(uint32_t profile, Fe2o3ProtectedProfileV1 *out);
int32_t fe2o3_protected_artifact_v1(uint32_t profile, Fe2o3ProtectedArtifactV1 *out);
int32_t fe2o3_protected_join_facts_v1(uint32_t profile, Fe2o3ProtectedJoinFactsV1 *out);
int32_t fe2o3_protected_validate_join_v1(const Fe2o3ProtectedJoinFactsV1 *facts,
                                         Fe2o3Slice1ErrorV1 *error);
/* Prepares the host request (`count` regions in role order) and joins it to
 * the profile's artifact.  `release_leases` and `device`: as for the LDS
 * GEMM join. */
int32_t fe2o3_protected_join_v1(uint32_t profile, const Fe2o3ProtectedRegionV1 *regions,
                                uint32_t count, int32_t device,
                                void (*release_leases)(void *user), void *user,
                                Fe2o3ProtectedLifecycleV1 **out, Fe2o3Slice1ErrorV1 *error);
int32_t fe2o3_protected_load_v1(Fe2o3ProtectedLifecycleV1 *lifecycle,
                                const Fe2o3Slice1AdapterV1 *adapter, Fe2o3Slice1ErrorV1 *error);
int32_t fe2o3_protected_dispatch_and_wait_v1(Fe2o3ProtectedLifecycleV1 *lifecycle,
                                             Fe2o3Slice1ErrorV1 *error);
/* COMPLETED only: terminal unload, receipt, handle freed. */
int32_t fe2o3_protected_unload_v1(Fe2o3ProtectedLifecycleV1 *lifecycle,
                                  Fe2o3ProtectedReceiptV1 *receipt);
void fe2o3_protected_release_v1(Fe2o3ProtectedLifecycleV1 *lifecycle);
int32_t fe2o3_protected_observe_v1(const Fe2o3ProtectedLifecycleV1 *lifecycle,
                                   Fe2o3Slice1ObservationV1 *out);

/* ---- collectives and workgroup synchronization ----------------------------------------- */

/* examples/wave64_collectives_v1/src/kernel.rs:18-67 (wave64_collectives_v1).
 * One wave64: lane l contributes input[l] if bit l of active_mask is set,
 * else +0.  Active lanes publish the full masked sum, the inclusive and the
 * exclusive prefix sums in physical lane order; inactive lanes publish +0
 * in all three.  The sum is six XOR-butterfly rounds and the scans six
 * Hillis-Steele rounds (examples/wave64_collectives_v1/src/oracle.rs:150-172),
 * so every bit matches the reference's oracle for any finite input.  All
 * four lengths 64. */
int32_t fe2o3_wave64_collectives_v1(const float *input, uint64_t input_len,
                                    uint64_t active_mask, float *reduction,
                                    uint64_t reduction_len, float *inclusive,
                                    uint64_t inclusive_len, float *exclusive,
                                    uint64_t exclusive_len, void *stream);

/* The same collectives over `rows` independent 64-element rows (row r =
 * elements 64r .. 64r+63, mask masks[r]); the reference has only the single
 * wave.  input/reduction/inclusive/exclusive rows*64, masks rows. */
int32_t fe2o3_wave64_collectives_rows(const float *input, uint64_t input_len,
                                      const uint64_t *masks, uint64_t masks_len,
                                      float *reduction, uint64_t reduction_len,
                                      float *inclusive, uint64_t inclusive_len,
                                      float *exclusive, uint64_t exclusive_len,
                                      uint64_t rows, void *stream);

/* examples/workgroup_sync_v1/src/kernel.rs:18-78 (lds_publish_read_reduce_i32_v1).
 * output[0] = sum of values[0..63]: each lane publishes one value to its own
 * LDS slot, uniform barriers around a halving tree, lane 0 writes.  The
 * addition wraps; the result is the exact sum whenever it fits in int32
 * (the reference admits only such inputs).  Lengths 64 and 1. */
int32_t fe2o3_lds_reduce_i32_v1(const int32_t *values, uint64_t values_len,
                                int32_t *output, uint64_t output_len, void *stream);

/* examples/workgroup_sync_v1/src/scoped_atomic.rs:11-32 (scoped_atomic_add_u32_v1).
 * For each lane l with eligible[l] != 0, one relaxed system-scope atomic
 * add of values[l] to *target (which keeps its prior contents as the
 * initial value).  Lengths 64; target 4-byte aligned. */
int32_t fe2o3_scoped_atomic_add_u32_v1(const uint32_t *values, uint64_t values_len,
                                       const uint32_t *eligible, uint64_t eligible_len,
                                       uint32_t *target, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* FE2O3_MI355X_H */
