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
 * writes the sentinel outputs its declaration states, marks the device's
 * contract-status word and exits normally; the next successful
 * fe2o3_rt_device_synchronize or fe2o3_rt_stream_synchronize on that device
 * returns FE2O3_ERR_NONFINITE and clears the word.  The word is per device,
 * like the reference's context-wide fault: a synchronize reports what any
 * kernel that finished before it on the device found, whichever stream
 * launched it.  Event synchronization does not read the word. */
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
 * lengths m*k, n*k, m*n.  Any m, n, k; the MFMA fast path needs m, n
 * multiples of 256, k a multiple of 64 and 16-byte aligned pointers. */
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
 * [batch, heads, seq].  head_dim must be 128; seq a multiple of 128 for the
 * MFMA path (other seq values are rejected with FE2O3_ERR_SHAPE). */
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
 * requested/admitted experts, offsets experts+1. */
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
 * accumulation; A row-major, B stored [n,k] (k contiguous).  m, n multiples
 * of 256, k a multiple of 128. */
int32_t fe2o3_gemm_fp8_nt(const uint8_t *a, uint64_t a_len, const uint8_t *b,
                          uint64_t b_len, const float *scale_a,
                          const float *scale_b, uint16_t *c, uint64_t c_len,
                          uint32_t m, uint32_t n, uint32_t k, void *stream);

/* crates/fe2o3-host/src/moe_routing_expert_bridge_v1.rs:220-389
 * (check_host_observed_moe_routing_output_v1) with the compact pack plan of
 * crates/fe2o3-host/src/generated_moe_expert_v1.rs:159-190, on the device
 * and for any tokens (at most 12288), experts (1..64) and capacity
 * (0xFFFFFFFF = unbounded).  Checks a complete routing output (the seven
 * arrays of fe2o3_moe_top2_route) and writes the reference's FIRST failing
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
 * index >= *count (0 for an unknown entry).  120-byte record. */
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
