/*
 * fe2o3_oracle.h -- CPU restatement of the reference's deterministic oracles
 * for the dense-compute path (tiled/scalar GEMM, flash attention, row softmax,
 * top-2 MoE router and expert pipeline) plus the oracles this build adds for
 * the scaled-up configurations (bf16 NT GEMM, OCP e4m3 GEMM, MoE SiLU FFN).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/, the
 * smoke() entry of __graft_entry__.py and bench.py's cpu_baseline leg may load
 * it.  The product library (fe2o3_amd/) never links or calls it.
 *
 * Arithmetic rules (all files are compiled with -ffp-contract=off, no
 * fast-math, SSE/AVX scalar semantics, FLT_EVAL_METHOD == 0):
 *   - every f32 product and sum is a separate round-to-nearest-even op,
 *     matching the reference's black_box'd helpers
 *     (examples/tiled_gemm_v1/src/oracle.rs:262-270);
 *   - OpenMP parallelism only splits independent output elements, so results
 *     are bit-identical for any thread count.
 *
 * Status codes: 0 = ok, negative = fail-closed rejection (outputs untouched).
 */
#ifndef FE2O3_ORACLE_H
#define FE2O3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  FE2O3O_OK = 0,
  FE2O3O_ERR_LENGTH = -2,        /* wrong slice length (WrongLength)        */
  FE2O3O_ERR_SHAPE = -3,         /* tile multiple / plan rejection          */
  FE2O3O_ERR_STRIDE = -4,        /* StrideTooSmall                          */
  FE2O3O_ERR_NONFINITE = -5,     /* NaN / inf input                         */
  FE2O3O_ERR_SUBNORMAL = -6,     /* subnormal input                         */
  FE2O3O_ERR_ALPHABET = -7,      /* outside the pinned BF16 alphabet        */
  FE2O3O_ERR_INTERMEDIATE = -8,  /* unsupported intermediate value          */
  FE2O3O_ERR_MISMATCH = -9,      /* comparison failed                       */
  FE2O3O_ERR_POLICY = -10,       /* malformed comparison policy             */
  FE2O3O_ERR_EMPTY = -11,        /* empty row                               */
  FE2O3O_ERR_TOO_LARGE = -12,    /* row above the bounded oracle maximum    */
  FE2O3O_ERR_NO_ACTIVE = -13,    /* mask removes every element              */
  FE2O3O_ERR_WEIGHTS = -14,      /* MoE route weight pair policy            */
  FE2O3O_ERR_ROUTING = -15,      /* routing record inconsistent             */
  FE2O3O_ERR_OVERFLOW = -16,     /* extent overflow                         */
  FE2O3O_ERR_SUM = -17,          /* softmax active sum outside policy       */
  FE2O3O_ERR_INFINITE = -18      /* infinite input (NaN uses ERR_NONFINITE) */
};

/* ---- numeric vocabulary (crates/fe2o3-device/src/half.rs:182-195) ------- */
uint16_t fe2o3o_bf16_from_f32(float value);
float fe2o3o_bf16_to_f32(uint16_t bits);
void fe2o3o_bf16_from_f32_array(const float *in, uint16_t *out, size_t n);
void fe2o3o_bf16_to_f32_array(const uint16_t *in, float *out, size_t n);

/* ---- reference input generator (examples/tiled_gemm_v1/src/inputs.rs) --- */
uint64_t fe2o3o_mix64(uint64_t value);
void fe2o3o_generate_inputs_v1(uint32_t m, uint32_t n, uint32_t k, uint64_t seed,
                               uint16_t *a, uint16_t *b);
/* Returns 0, or an error code with *operand (0=A,1=B) and *index set. */
int32_t fe2o3o_validate_evidence_inputs_v1(uint32_t m, uint32_t n, uint32_t k,
                                           const uint16_t *a, uint64_t a_len,
                                           const uint16_t *b, uint64_t b_len,
                                           int32_t *operand, uint64_t *index);

/* ---- this build's counter-based generators (bit-identical on the GPU) --- */
float fe2o3o_counter_normal(uint64_t seed, uint64_t domain, uint64_t index);
float fe2o3o_counter_uniform_pm1(uint64_t seed, uint64_t domain, uint64_t index);
void fe2o3o_fill_normal_bf16(uint16_t *out, uint64_t n, uint64_t seed,
                             uint64_t domain, float scale, uint64_t first_index);
void fe2o3o_fill_normal_f32(float *out, uint64_t n, uint64_t seed,
                            uint64_t domain, float scale, uint64_t first_index);
void fe2o3o_fill_uniform_f32(float *out, uint64_t n, uint64_t seed,
                             uint64_t domain, uint64_t first_index);

/* ---- GEMM oracles -------------------------------------------------------- */
/* examples/tiled_gemm_v1/src/oracle.rs:284-320 (row-major, C[M,N] f32). */
int32_t fe2o3o_tiled_gemm_arithmetic_v1(uint32_t m, uint32_t n, uint32_t k,
                                        const uint16_t *a, uint64_t a_len,
                                        const uint16_t *b, uint64_t b_len,
                                        float *c);
/* examples/tiled_gemm_v1/src/numerical_contract.rs:139-186 (GemmSpec). */
int32_t fe2o3o_gemm_spec_checked(uint64_t m, uint64_t n, uint64_t k,
                                 uint64_t lda, uint64_t ldb, uint64_t ldc,
                                 uint64_t *a_len, uint64_t *b_len,
                                 uint64_t *c_len);
/* numerical_contract.rs:310-341: C_out = alpha*(sum AB) + beta*C_in. */
int32_t fe2o3o_evaluate_source(uint64_t m, uint64_t n, uint64_t k,
                               uint64_t lda, uint64_t ldb, uint64_t ldc,
                               const uint16_t *a, uint64_t a_len,
                               const uint16_t *b, uint64_t b_len,
                               const float *c, uint64_t c_len, float alpha,
                               float beta, float *out);
/* numerical_contract.rs:536-721: strict finite-normal admission + evaluate. */
int32_t fe2o3o_build_hardware_expectation(uint64_t m, uint64_t n, uint64_t k,
                                          uint64_t lda, uint64_t ldb,
                                          uint64_t ldc, const uint16_t *a,
                                          uint64_t a_len, const uint16_t *b,
                                          uint64_t b_len, const float *c,
                                          uint64_t c_len, float alpha,
                                          float beta, float *out);
/* numerical_contract.rs:901-981.  policy 0 = ExactBits, 1 = Bounded.
 * report[0]=max_abs, report[1]=max_rel, *max_ulps, *bad_index on mismatch. */
int32_t fe2o3o_compare_hardware(const float *expected, const float *observed,
                                uint64_t n, int32_t policy, float max_abs,
                                float max_rel, uint32_t max_ulps, float *report,
                                uint32_t *max_ulp_error, uint64_t *bad_index);
uint32_t fe2o3o_ulp_distance(float left, float right);

/* examples/tiled_gemm_v1/src/general_reference.rs:171-268: tiled schedule
 * with zero-filled tails and XOR4 staging.  trace[6] = {workgroups,
 * reduction_phases, publish_barriers, reuse_barriers, a_zero_fills,
 * b_zero_fills}; trace[6]=output_stores, trace[7]=c_predicated_stores. */
int32_t fe2o3o_general_reference_v1(uint32_t m, uint32_t n, uint32_t k,
                                    uint32_t lda, uint32_t ldb, uint32_t ldc,
                                    const uint16_t *a, uint64_t a_len,
                                    const uint16_t *b, uint64_t b_len,
                                    const float *c, uint64_t c_len, float alpha,
                                    float beta, float *out, uint64_t *trace);
/* crates/fe2o3-device/src/tensor.rs:147-183 */
int32_t fe2o3o_row_major_xor4(uint32_t row, uint32_t col, uint32_t *physical);

/* examples/scalar_gemm_v1/src/harness.rs:87-112 */
void fe2o3o_scalar_gemm(uint32_t m, uint32_t n, uint32_t k, const float *a,
                        const float *b, float *c);
void fe2o3o_scalar_gemm_inputs(uint64_t a_len, uint64_t b_len, float *a,
                               float *b);

/* Same per-element recurrence as tiled_gemm_arithmetic_oracle_v1, evaluated
 * for rows [row_begin,row_end) of C = A * B^T with A row-major [M,K] and B
 * stored "column-major" ([N,K], K contiguous).  Output f32 [rows, N]. */
void fe2o3o_gemm_bf16_nt_rows(uint32_t m, uint32_t n, uint32_t k,
                              const uint16_t *a, const uint16_t *b,
                              uint32_t row_begin, uint32_t row_end, float *out,
                              int32_t threads);
/* Sampled outputs (row[i], col[i]) of the same recurrence. */
void fe2o3o_gemm_bf16_nt_points(uint32_t k, const uint16_t *a_rows,
                                const uint16_t *b_cols, uint64_t points,
                                float *out, int32_t threads);
/* scalar_gemm recurrence on rows [row_begin,row_end) of row-major f32 A[M,K],
 * B[K,N]. */
void fe2o3o_gemm_f32_rows(uint32_t m, uint32_t n, uint32_t k, const float *a,
                          const float *b, uint32_t row_begin, uint32_t row_end,
                          float *out, int32_t threads);

/* ---- flash attention ----------------------------------------------------- */
/* examples/flash_attention_v1/src/oracle.rs:222-284 (fixed B1/H1/N8/D16,
 * causal, scale 0.25).  row_maxima/denominators may be NULL. */
int32_t fe2o3o_flash_attention_v1(const float *q, uint64_t q_len,
                                  const float *k, uint64_t k_len,
                                  const float *v, uint64_t v_len, float *out,
                                  uint64_t out_len, double *row_maxima,
                                  double *row_denominators);
/* Same two-pass f64 reference generalised to [B,H,S,D] bf16 tensors for the
 * listed (bh, query) rows.  out is [rows, D] f32, lse is [rows] f32
 * (natural log: max + ln(denominator)). */
int32_t fe2o3o_flash_attention_rows_bf16(const uint16_t *q, const uint16_t *k,
                                         const uint16_t *v, uint32_t s,
                                         uint32_t d, int32_t causal,
                                         float scale, const uint32_t *bh,
                                         const uint32_t *rows, uint64_t count,
                                         float *out, float *lse,
                                         int32_t threads);

/* ---- row softmax --------------------------------------------------------- */
/* examples/row_softmax_v1/src/numerical_contract.rs:130-199 (f64 oracle).
 * mask may be NULL; state = {maximum(f32 as double), denominator, active}. */
int32_t fe2o3o_row_softmax_oracle_v1(const float *input, uint64_t len,
                                     const uint8_t *mask, float *out,
                                     double *state);
/* numerical_contract.rs:201-257. */
int32_t fe2o3o_compare_row_softmax_v1(const float *expected,
                                      const float *actual, uint64_t len,
                                      const uint8_t *mask, float abs_tol,
                                      float rel_tol, float sum_tol,
                                      uint32_t max_ulps, uint64_t *bad_index);
/* examples/row_softmax_v1/src/lib.rs:121-159 (f32 host reference, 64 wide). */
int32_t fe2o3o_row_softmax_reference_v1(const float *input, float *out);
/* Many rows of fe2o3o_row_softmax_oracle_v1 (no mask), OpenMP over rows. */
int32_t fe2o3o_row_softmax_rows(const float *input, uint64_t rows,
                                uint64_t cols, float *out, int32_t threads);
/* Each row of `actual` against fe2o3o_row_softmax_oracle_v1 of the same row
 * of `input` under fe2o3o_compare_row_softmax_v1's policy, OpenMP over rows;
 * stats[5] = {failing rows, first failing row (rows if none), max abs
 * difference, max |oracle|, max |f64 row sum - 1|}. */
int32_t fe2o3o_row_softmax_check_rows(const float *input, const float *actual,
                                      uint64_t rows, uint64_t cols, float abs_tol,
                                      float rel_tol, float sum_tol, uint32_t max_ulps,
                                      int32_t threads, double *stats);

/* ---- MoE top-2 router ---------------------------------------------------- */
#define FE2O3O_DROP_ROUTE 0xffffffffu
/* examples/moe_top2_v1/src/oracle.rs:63-143 generalised to T tokens and E
 * experts (sort-based selector).  capacity = 0xffffffff means unbounded.
 * Output arrays: top2[2T], requested[E], admitted[E], offsets[E+1],
 * route_slots[2T], permutation[2T], inverse[2T]. */
int32_t fe2o3o_moe_top2_route(const float *logits, uint32_t tokens,
                              uint32_t experts, uint32_t capacity,
                              uint32_t *top2, uint32_t *requested,
                              uint32_t *admitted, uint32_t *offsets,
                              uint32_t *route_slots, uint32_t *permutation,
                              uint32_t *inverse);
/* examples/moe_top2_v1/src/kernel.rs:25-59 running selector (the reference's
 * second, independent implementation).  out[2]. */
void fe2o3o_moe_select_top2_running(const float *logits_row, uint32_t experts,
                                    uint32_t *out);
/* Gating weights for the selected pair: w0 = 1/(1+exp(l1-l0)), w1 = 1-w0,
 * so every pair sums to exactly 1.0f (examples/moe_expert_v1/src/pipeline.rs
 * :137-148 requires that). */
void fe2o3o_moe_top2_weights(const float *logits, uint32_t tokens,
                             uint32_t experts, const uint32_t *top2,
                             float *weights);

/* examples/moe_expert_v1/src/oracle.rs:32-90 (T8/E4/H16/O16 fixed profile,
 * routing from fe2o3o_moe_top2_route with capacity 4). */
int32_t fe2o3o_moe_expert_independent_v1(
    const float *logits, const uint16_t *activations, uint64_t act_len,
    const uint16_t *weights, uint64_t w_len, const float *route_weights,
    uint64_t rw_len, const uint32_t *top2, const uint32_t *offsets,
    const uint32_t *inverse, float *expert_tiles, float *compact,
    float *combined, float *route_output);
/* examples/moe_expert_v1/src/pipeline.rs:166-270 (host schedule model). */
int32_t fe2o3o_moe_expert_pipeline_v1(
    const float *logits, const uint16_t *activations, uint64_t act_len,
    const uint16_t *weights, uint64_t w_len, const float *route_weights,
    uint64_t rw_len, const uint32_t *top2, const uint32_t *admitted,
    const uint32_t *offsets, const uint32_t *permutation,
    const uint32_t *inverse, uint16_t *activation_tiles, float *expert_tiles,
    float *compact, float *combined);

/* Config-5 SiLU expert FFN for one route (not in the reference; closed form
 * silu(x) = x / (1 + exp(-x))).  x[H] bf16; w_gate,w_up [F,H] bf16 (H
 * contiguous); w_down [H,F] bf16 (F contiguous).  hidden[F] receives the
 * bf16-rounded activation, y[H] the f32 expert output. */
void fe2o3o_moe_ffn_route(const uint16_t *x, const uint16_t *w_gate,
                          const uint16_t *w_up, const uint16_t *w_down,
                          uint32_t h, uint32_t f, uint16_t *hidden, float *y);
/* The same for n (token, expert) pairs, OpenMP over pairs (hidden not
 * kept): x [tokens, H]; weights as above with a leading expert index;
 * y [n, H]. */
void fe2o3o_moe_ffn_routes(const uint16_t *x, const uint16_t *w_gate,
                           const uint16_t *w_up, const uint16_t *w_down,
                           uint32_t h, uint32_t f, const uint32_t *tokens,
                           const uint32_t *experts, uint64_t n, float *y,
                           int32_t threads);

/* ---- OCP FP8 E4M3FN ------------------------------------------------------ */
uint8_t fe2o3o_fp8e4m3_from_f32(float value);
float fe2o3o_fp8e4m3_to_f32(uint8_t bits);
/* gfx942 FNUZ fp8 (format 0 = E4M3, 1 = E5M2): crates/fe2o3-device/src/fp8.rs:296-381 */
uint8_t fe2o3o_fnuz_from_f32_bits(uint32_t bits, int32_t format);
uint32_t fe2o3o_fnuz_to_f32_bits(uint8_t q, int32_t format);
void fe2o3o_fnuz_from_f32_array(const float *x, uint64_t n, int32_t format, uint8_t *q);
float fe2o3o_amax_f32(const float *x, uint64_t n, int32_t threads);
void fe2o3o_quantize_e4m3(const float *x, uint64_t n, float scale,
                          uint8_t *out, int32_t threads);
/* Sampled outputs of C = (sa*sb) * (A_q * B_q^T), A row-major [., K],
 * B [N,K]; returns bf16 bits and the f32 value before narrowing. */
void fe2o3o_gemm_fp8_points(uint32_t k, const uint8_t *a_rows,
                            const uint8_t *b_cols, uint64_t points,
                            float scale_ab, float *out_f32, uint16_t *out_bf16,
                            int32_t threads);
/* Whole rows of the same product (f32 values before narrowing). */
void fe2o3o_gemm_fp8_nt_rows(uint32_t n, uint32_t k, const uint8_t *a, const uint8_t *b,
                             float scale_ab, uint32_t row_begin, uint32_t row_end,
                             float *out_f32, int32_t threads);

/* ---- collectives, workgroup sync, routing consistency (sync.c) ---- */

void fe2o3o_wave64_collectives_compute(const float *input, uint64_t mask, float *reduction,
                                       float *inclusive, float *exclusive);
int32_t fe2o3o_wave64_collectives_v1(const float *input, uint64_t mask, float *reduction,
                                     float *inclusive, float *exclusive);
int32_t fe2o3o_lds_reduce_i32_v1(const int32_t *values, int32_t *output);
int32_t fe2o3o_atomic_add_u32_v1(uint32_t initial, const uint32_t *values,
                                 const uint32_t *eligible, uint32_t *result);

/* Routing consistency record kinds, in the order the reference checks them
 * (crates/fe2o3-host/src/moe_routing_expert_bridge_v1.rs:67-140); record =
 * {kind, index, expected, actual}:
 *   EXPERT_OUT_OF_RANGE   index route, actual expert
 *   DUPLICATE_TOKEN_EXPERT index token, actual expert
 *   REQUESTED_COUNT       index expert, expected, actual
 *   CAPACITY              index expert, actual admitted
 *   ADMITTED_COUNT        index expert, expected, actual
 *   FIRST_OFFSET          actual offsets[0]
 *   NONMONOTONE_OFFSETS   index expert, expected = start, actual = end
 *   OFFSET_MISMATCH       index expert + 1, expected, actual
 *   PLAN_OFFSET_ORDER     index expert, actual end        (compact pack plan)
 *   PLAN_CAPACITY         index expert, actual rows       (compact pack plan)
 *   SLOT_OUT_OF_RANGE     index route, expected = accepted routes, actual slot
 *   DUPLICATE_SLOT        index route, actual slot
 *   STABLE_SLOT           index route, expected, actual
 *   INVERSE               index route, expected, actual
 *   PERMUTATION           index slot, expected route, actual permutation[slot]
 *   PREFIX_HOLE           index slot
 *   PERMUTATION_ROUTE     index slot, actual route
 *   PERMUTATION_TAIL      index slot, actual */
enum {
  FE2O3O_RC_OK = 0,
  FE2O3O_RC_EXPERT_OUT_OF_RANGE = 1,
  FE2O3O_RC_DUPLICATE_TOKEN_EXPERT = 2,
  FE2O3O_RC_REQUESTED_COUNT = 3,
  FE2O3O_RC_CAPACITY = 4,
  FE2O3O_RC_ADMITTED_COUNT = 5,
  FE2O3O_RC_FIRST_OFFSET = 6,
  FE2O3O_RC_NONMONOTONE_OFFSETS = 7,
  FE2O3O_RC_OFFSET_MISMATCH = 8,
  FE2O3O_RC_PLAN_OFFSET_ORDER = 9,
  FE2O3O_RC_PLAN_CAPACITY = 10,
  FE2O3O_RC_SLOT_OUT_OF_RANGE = 11,
  FE2O3O_RC_DUPLICATE_SLOT = 12,
  FE2O3O_RC_STABLE_SLOT = 13,
  FE2O3O_RC_INVERSE = 14,
  FE2O3O_RC_PERMUTATION = 15,
  FE2O3O_RC_PREFIX_HOLE = 16,
  FE2O3O_RC_PERMUTATION_ROUTE = 17,
  FE2O3O_RC_PERMUTATION_TAIL = 18
};
int32_t fe2o3o_moe_routing_check(const uint32_t *top2, const uint32_t *requested,
                                 const uint32_t *admitted, const uint32_t *offsets,
                                 const uint32_t *slots, const uint32_t *permutation,
                                 const uint32_t *inverse, uint32_t tokens, uint32_t experts,
                                 uint32_t capacity, uint32_t *record);

#ifdef __cplusplus
}
#endif
#endif
