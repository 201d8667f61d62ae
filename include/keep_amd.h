/*
 * keep_amd -- C ABI of the MI355X (gfx950) routed E8P expert path.
 *
 * Every entry point takes caller-owned device pointers, explicit shapes and a
 * hipStream_t (passed as void*), allocates no device memory, validates its
 * arguments on the host before any launch and returns 0 or a negative
 * KEEP_E* code; keep_last_error() then holds a message (thread-local).
 *
 * Dtype enums: KEEP_F32 = 0, KEEP_F16 = 1, KEEP_BF16 = 2.
 * Index arrays are int32. Codes are uint16 (E8P, code_bits = 16) or uint8
 * (E8 1-bit table, code_bits = 8). Codebooks are the packed uint32[256]
 * nibble tables of the reference (src/keep/vq/e8.py:127-139, :169-179).
 * A route index outside [0, num_experts) never faults: that route's output
 * row is written as NaN.
 */
#ifndef KEEP_AMD_H
#define KEEP_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { KEEP_F32 = 0, KEEP_F16 = 1, KEEP_BF16 = 2 };
enum { KEEP_OK = 0, KEEP_EINVAL = -1, KEEP_ELAUNCH = -2, KEEP_EUNSUPPORTED = -3 };
enum { KEEP_SCORE_SOFTMAX = 0, KEEP_SCORE_SIGMOID = 1, KEEP_SCORE_SQRTSOFTPLUS = 2 };

/* Message of the last failed call on this thread ("" if none). */
const char* keep_last_error(void);
/* ABI version (bumped on any signature change). */
int keep_abi_version(void);

/* Host-side: the E8P packed absolute table, uint32[256], built from its closed
 * form. Replaces keep.vq.e8.e8p_packed_abs_grid (src/keep/vq/e8.py:127-139). */
int keep_e8p_packed_abs_grid(uint32_t* out256);
/* Host-side: the packed 8-bit E8 residual table, uint32[256].
 * Replaces keep.vq.e8.e8_1bit_packed (src/keep/vq/e8.py:169-179). */
int keep_e8_1bit_packed(uint32_t* out256);

/* Decode n E8P codewords to float32 [n, 8], optionally times per-group scales
 * (scales != NULL: codes viewed as rows of codewords_per_row codewords, one
 * scale per group_codewords consecutive codewords). Bit-exact with
 * keep.vq.e8.decode_e8p / decode_weight_matrix (src/keep/vq/e8.py:210-234,
 * :542-571). */
int keep_e8p_decode(const uint16_t* codes, int64_t n, const uint32_t* table,
                    const void* scales, int scale_dtype, int64_t codewords_per_row,
                    int64_t group_codewords, float* out, void* stream);
/* 8-bit E8 decode (code_bits = 8): code byte c indexes the packed table
 * (nibble d = dim d, value (nibble - 8) / 2), times the same optional group
 * scales. Replaces decode_e8_1bit / decode_weight_matrix(code_bits=8)
 * (src/keep/vq/e8.py:542-571). */
int keep_e8_1bit_decode(const uint8_t* codes, int64_t n, const uint32_t* table, const void* scales,
                        int scale_dtype, int64_t codewords_per_row, int64_t group_codewords, float* out,
                        void* stream);

/* Nearest-codeword encoder: codes[i] = the codeword (code_bits 16: E8P uint16
 * of the packed abs table; 8: the 8-bit E8 uint8 index of the packed E8
 * table) nearest to vector i (fp32 [n, 8], divided by scales[i /
 * vectors_per_scale] when scales is non-null, the quotient correctly rounded
 * to fp32) under the diagonal metric diagonal (diag_mode 0: none; 1: one
 * shared [8]; 2: one [8] per vector): the minimiser of
 * ((q0+q1)+(q2+q3))+((q4+q5)+(q6+q7)), q_d = w_d (v_d - c_d)^2 in double,
 * ties to the lowest code, as the exhaustive scan. The E8P search is factored
 * (2 shifts x 256 abs rows with the sign-parity fix).
 * Replaces encode_e8p_rtn / encode_e8p_rtn_diagonal_hessian
 * (src/keep/vq/e8.py:367-539), encode_e8_1bit_rtn (:283-287) and the RTN
 * search of quantize_weight_rtn (src/keep/quant/rtn.py:299-310). */
int keep_vq_encode(const float* vectors, int64_t n, int code_bits, const float* diagonal, int diag_mode,
                   const uint32_t* table, const float* scales, int64_t vectors_per_scale, void* codes,
                   void* stream);
/* scales[g] = max |x[g * group_size + j]| / divisor (fp32, correctly rounded)
 * over groups_total contiguous groups: the max_abs scale estimator of
 * src/keep/quant/rtn.py:253-264. */
int keep_group_absmax(const float* x, int64_t groups_total, int64_t group_size, float divisor, float* scales,
                      void* stream);

/* Routed VQ mat-vec: out[r, :] = W[rhs[r]] . x[row(r), :] for r < routes,
 * row(r) = lhs ? lhs[r] : r / x_div. W[e] is [N, K] given by codes [E, N, K/8]
 * and scales [E, N, K/group_size]. fp32 accumulate. rhs may be NULL when
 * num_experts == 1 (a single matrix: every route reads W[0], with no load of
 * a route vector before the code loads).
 * Optional nested residual (res_codes != NULL): 8-bit E8 codes [H, N, K/8],
 * res_scales [H, N, K/res_group_size], res_table = half2 pairs uint32[256*4]
 * (fp16 bits of dims 2k | 2k+1 << 16) and hot_of_slot[E] (row in the residual
 * arrays or 0xFFFFFFFF); base and residual accumulate separately.
 * Replaces ramp.kernels.e8p_m1.e8p_m1_token_layout / e8p_m1_per_route
 * (src/ramp/kernels/e8p_m1.py:134-183), e8p_nested_m1_* (e8p_nested_m1.py:90-112),
 * vq_qmv (vq_qmv.py:163-232, routes = 1), vq_qmm (vq_qmm.py:93-152) and the
 * direct / per_route_decoded branches of gather_vqmm (src/ramp/ops/vq_switch.py:916-1221). */
int keep_vq_matvec(const void* x, int x_dtype, int64_t x_rows,
                   const void* codes, int code_bits, const void* scales, int scale_dtype,
                   const uint32_t* table,
                   const int32_t* rhs, const int32_t* lhs, int64_t routes, int64_t x_div,
                   int64_t num_experts, int64_t N, int64_t K, int64_t group_size,
                   const uint8_t* res_codes, const void* res_scales, int64_t res_group_size,
                   const uint32_t* res_table, const uint32_t* hot_of_slot, int64_t num_hot,
                   void* out, int out_dtype, void* stream);

/* The residual tier alone: out[r, :] = W[rhs[r]] . x[r / x_div, :] for 8-bit E8
 * codes [E, N, K/8] with scales [E, N, K/group_size] and the packed E8 table
 * (nibble d = dim d); a route whose index is 0xFFFFFFFF writes zeros (any other
 * out-of-range index: NaN). fp32 accumulate. Replaces
 * ramp.kernels.e8_1bit_m1.e8_1bit_m1_token_layout / e8_1bit_m1_per_route
 * (src/ramp/kernels/e8_1bit_m1.py:48-97, e8_1bit_m1.metal:1-90). */
int keep_e8_1bit_matvec(const void* x, int x_dtype, int64_t x_rows, const uint8_t* codes, const void* scales,
                        int scale_dtype, const uint32_t* table, const uint32_t* rhs, int64_t routes,
                        int64_t x_div, int64_t num_experts, int64_t N, int64_t K, int64_t group_size, void* out,
                        int out_dtype, void* stream);

/* Expert-grouped verify rows: each tile holds up to m_rows routes of one
 * expert (tile_offset/tile_count index the sorted routes; tile_expert is
 * the expert). Routes of a tile share every code load and decode. Output row
 * sorted_route is written at out[sorted_route] (sorted order). Bit-identical
 * per route with keep_vq_matvec (same lane accumulation order). code_bits 8:
 * uint8 codes indexing a packed 8-bit E8 table (nibble d = dim d, value
 * (nibble - 8) / 2), the reference verify kernel's format; 16: E8P uint16.
 * Replaces gather_vqmm_verify_rows (src/ramp/ops/vq_switch.py:286-377) and
 * its kernel gather_vqmm_verify_mrows (src/ramp/kernels/gather_vqmm.py:287-419). */
int keep_vq_matvec_tiles(const void* x, int x_dtype, int64_t x_rows,
                         const void* codes, int code_bits, const void* scales, int scale_dtype,
                         const uint32_t* table, const int32_t* sorted_lhs, int64_t routes,
                         const int32_t* tile_expert, const int32_t* tile_offset,
                         const int32_t* tile_count, int64_t n_tiles, int64_t m_rows,
                         int64_t num_experts, int64_t N, int64_t K, int64_t group_size,
                         void* out, int out_dtype, void* stream);

/* Residency-biased dual top-k router, one evaluation per token:
 * scores = score_func(logits[T, E]); served idx/w = top-k of scores + bias_served
 * (an expert with bias_served <= -1e30 is absent: weight 0 if picked), weights
 * renormalised (if renormalize) and times route_scale; demand want/want_score =
 * top-k of scores + bias_demand with raw scores; admit[t, j] = want absent and
 * its normalised demand weight >= tau. Ties: larger key, then lower index.
 * bias_* may be NULL (zeros); want/want_score/admit may be NULL.
 * slot_map (int32 [E], NULL: none): the pool holds num_slots rows, expert e in
 * row slot_map[e]; the served idx are then rows (-1 for an entry outside
 * [0, num_slots)), as the serving router writes slot_of[chosen] (the demand
 * outputs stay expert ids). Callers map absent experts to any row (their
 * weight is 0); the same holds for every routed layer below that takes a
 * slot map, whose pools (codes, scales, hot_of_slot) are then per row.
 * Replaces MoEGate._expert_select (src/ramp/models/deepseek_v4_flash_adapter.py:923-940),
 * gate_masked (scripts/runpod/v41_reap/local_eval.py:69-91) and the dual top-k
 * kernel _TOPK (scripts/v41_build/omlx_lattice.py:77-97). */
int keep_router_dual_topk(const float* logits, int64_t T, int64_t E, int64_t k,
                          const float* bias_served, const float* bias_demand,
                          int score_func, int renormalize, float route_scale, float tau,
                          const int32_t* slot_map, int64_t num_slots,
                          int32_t* idx, float* w, int32_t* want, float* want_score,
                          uint8_t* admit, void* stream);

/* Device route plan: stable sort of routes by expert, its inverse, per-expert
 * counts/offsets and tile descriptors of at most `tile` routes (tiles in
 * expert order; entries past the last real tile have count 0, offset 0).
 * n_tiles_out[0] receives the real tile count. Buffers: order/inverse [R],
 * counts/offsets [E], tile_* [max_tiles], max_tiles >= ceil(R/tile) + E.
 * Replaces argsort + _inverse_permutation + _expert_block_tile_descriptors
 * (src/ramp/ops/vq_switch.py:100-152) and _verify_row_tile_descriptors (:186-225). */
int keep_route_plan(const int32_t* rhs, int64_t R, int64_t E, int64_t tile,
                    int32_t* order, int32_t* inverse, int32_t* counts, int32_t* offsets,
                    int32_t* tile_expert, int32_t* tile_offset, int32_t* tile_count,
                    int64_t max_tiles, int32_t* n_tiles_out, void* stream);

/* Decode tables for the matrix-core kernels, built on the device from the
 * 256-entry packed abs grid: at offset 0 the 4 KiB int8 T / M tables (T[idx]:
 * the 8 bytes 4 x the unsigned even-parity codeword; M[signs]: its sign and
 * parity mask, so a codeword's int8 weights x 4 are T[idx] ^ M[signs],
 * src/keep/vq/e8.py:203-234), then a 256-byte word that is nonzero when the
 * grid holds a value those tables cannot express (the kernels then write
 * NaN), then the 64 KiB LDS image of T and M (256 rows of sixteen copies)
 * that the int8 kernels stage per block: 69,888 bytes in all. `prepared` must hold keep_e8p_prepared_bytes() bytes. No reference
 * counterpart: it replaces the per-threadgroup half2 pair decode of
 * src/ramp/kernels/e8p_m1.metal:36-45 at a larger scale. */
int keep_e8p_prepare(const uint32_t* table, void* prepared, void* stream);
int keep_e8p_prepared_bytes(void);

/* Fused routed SwiGLU MoE for few tokens (decode / verify), any shape:
 * h[t, j, :] = swiglu(Wg[e] x_t, Wu[e] x_t) (clamped by swiglu_limit if > 0),
 * out[t, :] = sum_j w[t, j] * Wd[e] h[t, j, :], e = idx[t, j].
 * Gate/up codes [E, I, H/8], down codes [E, H, I/8]; h_work is caller-provided
 * [T * k * I] bf16 (SwiGLU in fp32, stored as bf16 as the reference's serving
 * step stores it; fp16 would overflow), in natural [T, k, I] order. Two
 * launches on `stream` of the packed-table mat-vec kernels (H and I multiples
 * of 8, scale groups of 8-element multiples); `prepared` is accepted and not
 * read. The shapes keep_moe_tiles serves (T <= 256, H and I multiples of 256)
 * run faster there; keep_amd.moe_decode picks between the two.
 * Replaces QuantizedVQSwitchGLU.__call__ (src/ramp/models/glm4_moe_adapter.py:367-372)
 * plus the weighted combine of DeepseekV4FlashVQMoE.__call__
 * (src/ramp/models/deepseek_v4_flash_adapter.py:1776-1784) and the decode step
 * of scripts/v41_build/omlx_lattice.py:359-371. */
int keep_moe_decode(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I,
                    const int32_t* idx, const float* w, int64_t k, int64_t num_experts,
                    const uint16_t* gate_codes, const void* gate_scales,
                    const uint16_t* up_codes, const void* up_scales,
                    const uint16_t* down_codes, const void* down_scales, int scale_dtype,
                    int64_t group_size_h, int64_t group_size_i, const uint32_t* table,
                    const void* prepared, float swiglu_limit, void* h_work, void* out,
                    int out_dtype, void* stream);

/* The two launches of keep_moe_decode as separate entry points (same kernels,
 * same arguments): gate/up/SwiGLU into h_work, then down + weighted combine
 * from h_work (h_dtype must be KEEP_BF16). A route with
 * weight 0 is skipped by both. Replace the e8p_m1_token_layout gate/up pair
 * and the e8p_m1_per_route down + fp32 sum of scripts/v41_build/omlx_lattice.py:366-371. */
int keep_moe_gateup(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I,
                    const int32_t* idx, const float* w, int64_t k, int64_t num_experts,
                    const uint16_t* gate_codes, const void* gate_scales,
                    const uint16_t* up_codes, const void* up_scales, int scale_dtype,
                    int64_t group_size_h, const uint32_t* table, const void* prepared,
                    float swiglu_limit, void* h_work, void* stream);
int keep_moe_down(int h_dtype, int64_t T, int64_t H, int64_t I,
                  const int32_t* idx, const float* w, int64_t k, int64_t num_experts,
                  const uint16_t* down_codes, const void* down_scales, int scale_dtype,
                  int64_t group_size_i, const uint32_t* table, const void* prepared,
                  const void* h_work, void* out, int out_dtype, void* stream);

/* One routed MoE decode layer for one token in two launches on `stream`:
 * first the router (as keep_router_dual_topk with T = 1; outputs written to
 * idx/w/want/want_score/admit, the last three optional) fused with
 * gate/up/SwiGLU into h_work, then down + weighted combine into out[H], both
 * on the int8 matrix cores. No state is kept between calls. `prepared` is keep_e8p_prepare of the E8P
 * table. Serves H = 4096, I a multiple of 512 up to 2048, k <= 8, E <= 1024
 * and scale groups of 256-element multiples (keep_moe_layer_supported).
 * Replaces the serving decode step of scripts/v41_build/omlx_lattice.py:327-371
 * (router, gate/up, SwiGLU, down, fp32 combine) for batch 1. */
int keep_moe_layer_supported(int64_t num_experts, int64_t H, int64_t I, int64_t k,
                             int64_t group_size_h, int64_t group_size_i);
int keep_moe_layer(const float* logits, const float* bias_served, const float* bias_demand,
                   int score_func, int renormalize, float route_scale, float tau,
                   const int32_t* slot_map, int64_t num_slots,
                   int64_t num_experts, int64_t k, const void* x, int x_dtype, int64_t H, int64_t I,
                   const uint16_t* gate_codes, const void* gate_scales,
                   const uint16_t* up_codes, const void* up_scales,
                   const uint16_t* down_codes, const void* down_scales, int scale_dtype,
                   int64_t group_size_h, int64_t group_size_i, const void* prepared,
                   float swiglu_limit, int32_t* idx, float* w, int32_t* want, float* want_score,
                   uint8_t* admit, void* h_work, void* out, int out_dtype, void* stream);

/* keep_moe_layer without h_work: it allocates nothing and takes no
 * workspace. No counterpart in the reference; it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). h lives in a static device array of
 * 12,288 bf16 values (24 KiB, one copy per GPU for the life of the process),
 * so k * I <= 12288 (every shape keep_moe_layer serves); larger k * I returns
 * KEEP_EINVAL. Calls that overlap on one GPU (on different streams) share
 * that array and race; calls in one stream's order do not. Same outputs as
 * keep_moe_layer, bit for bit. */
int keep_moe_layer_noalloc(const float* logits, const float* bias_served, const float* bias_demand,
                           int score_func, int renormalize, float route_scale, float tau,
                           const int32_t* slot_map, int64_t num_slots,
                           int64_t num_experts, int64_t k, const void* x, int x_dtype, int64_t H, int64_t I,
                           const uint16_t* gate_codes, const void* gate_scales,
                           const uint16_t* up_codes, const void* up_scales,
                           const uint16_t* down_codes, const void* down_scales, int scale_dtype,
                           int64_t group_size_h, int64_t group_size_i, const void* prepared,
                           float swiglu_limit, int32_t* idx, float* w, int32_t* want, float* want_score,
                           uint8_t* admit, void* out, int out_dtype, void* stream);

/* The same layer in ONE launch of 256 blocks (one per compute unit, all
 * resident together): the router, gate/up/SwiGLU and down + combine, with
 * the whole code stream (gate/up, then down) requested as soon as a block has
 * routed the token. SwiGLU outputs pass between blocks through `workspace`
 * as tagged words: keep_moe_layer1_workspace_bytes(k, I) bytes, 256-byte
 * aligned, zero-filled before its first use and then handed unchanged to
 * every call on the same stream (it holds the call counter; calls that
 * overlap on one workspace race). A wait on another block that outlasts
 * ~200 us gives up: the outputs of the blocks that waited are NaN and
 * keep_moe_layer1_status() reports bit 1 (zero the workspace before the next
 * call). Each block issues its gate/up loads on routes chosen from the logit
 * order, certified equal to the exact selection or checked against it (and
 * reloaded) before use; a certified route found different would make that
 * block's outputs NaN and set status value 2 (never expected: a broken
 * certificate). Needs a device of at least 256 compute units. h is split into two
 * int8 terms per 256-wide slice, as in keep_moe_layer. Serves H = 4096, I
 * in {512, 1024, 1536, 2048}, k <= 8, E <= 1024, scale groups of
 * 256-element multiples. Replaces the serving decode step of
 * scripts/v41_build/omlx_lattice.py:327-371 for batch 1. */
int64_t keep_moe_layer1_workspace_bytes(int64_t k, int64_t I);
int keep_moe_layer1_status(const void* workspace, uint32_t* status, void* stream);
/* The give-up budget of every later keep_moe_layer1 launch in this process,
 * in ticks of the GPU's 100 MHz real-time counter (default 20000 = 200 us,
 * at most 1e8 = 1 s); *previous (if not null) receives the old value. A
 * launch whose wait for another block's h outlasts it writes NaN for the
 * routes that wave holds and sets status bit 1: callers check
 * keep_moe_layer1_status() where a NaN output must not pass unnoticed. Tests
 * use a budget of 0 to drive the give-up path. No counterpart in the
 * reference (its decode step has no cross-block wait). */
int keep_moe_layer1_set_spin_ticks(uint32_t ticks, uint32_t* previous);
int keep_moe_layer1(const float* logits, const float* bias_served, const float* bias_demand,
                    int score_func, int renormalize, float route_scale, float tau,
                    const int32_t* slot_map, int64_t num_slots,
                    int64_t num_experts, int64_t k, const void* x, int x_dtype, int64_t H, int64_t I,
                    const uint16_t* gate_codes, const void* gate_scales,
                    const uint16_t* up_codes, const void* up_scales,
                    const uint16_t* down_codes, const void* down_scales, int scale_dtype,
                    int64_t group_size_h, int64_t group_size_i, const void* prepared,
                    float swiglu_limit, int32_t* idx, float* w, int32_t* want, float* want_score,
                    uint8_t* admit, void* workspace, int64_t workspace_bytes, void* out, int out_dtype,
                    void* stream);

/* keep_moe_layer1 with the nested 3-bit tier: an expert's pool row with a
 * residual row (hot_of_slot[row] < num_hot; 0xFFFFFFFF = none; any other value
 * makes that route's output NaN) adds R[row] . x to gate and up and R[row] . h
 * to down, R the 8-bit E8 residual (codes uint8 [num_hot, N, K/8] indexing
 * res_table, the packed E8 table uint32[256], value (nibble - 8) / 2 per
 * dimension, times scales [num_hot, N, K/group] of res_scale_dtype; residual
 * groups of 256-element multiples). Same workspace, give-up budget and status
 * as keep_moe_layer1; with a slot map, num_slots <= num_experts. Replaces the
 * decode step with the tier, scripts/v41_build/omlx_lattice.py:327-371
 * (nested mat-vecs 358-370, e8p_nested_m1.py:90-112), in one launch. */
int keep_moe_layer1_nested(const float* logits, const float* bias_served, const float* bias_demand,
                           int score_func, int renormalize, float route_scale, float tau,
                           const int32_t* slot_map, int64_t num_slots, int64_t num_experts, int64_t k,
                           const void* x, int x_dtype, int64_t H, int64_t I,
                           const uint16_t* gate_codes, const void* gate_scales,
                           const uint16_t* up_codes, const void* up_scales,
                           const uint16_t* down_codes, const void* down_scales, int scale_dtype,
                           int64_t group_size_h, int64_t group_size_i, const void* prepared,
                           float swiglu_limit, int32_t* idx, float* w, int32_t* want, float* want_score,
                           uint8_t* admit, void* workspace, int64_t workspace_bytes, void* out, int out_dtype,
                           const uint32_t* hot_of_slot, int64_t num_hot,
                           const uint8_t* res_gate_codes, const void* res_gate_scales,
                           const uint8_t* res_up_codes, const void* res_up_scales,
                           const uint8_t* res_down_codes, const void* res_down_scales, int res_scale_dtype,
                           int64_t res_group_size_h, int64_t res_group_size_i, const uint32_t* res_table,
                           void* stream);

/* keep_moe_layer with the nested 3-bit tier: an expert e with a residual row
 * (hot_of_slot[e] < num_hot; 0xFFFFFFFF = none; any other value makes that
 * route's output NaN) adds R[row] . x to gate, up and down, R the 8-bit E8
 * residual (codes uint8 [num_hot, N, K/8] indexing the packed E8 table,
 * value (nibble - 8) / 2 per dimension, times scales [num_hot, N, K/group]
 * of res_scale_dtype; residual groups of 256-element multiples). res_image
 * is the residual table's LDS image (keep_e8_1bit_image, once per table);
 * hot_route is device scratch of k int32 handed from the first launch to the
 * second. Same two launches as keep_moe_layer, which stays as it is.
 * Replaces the decode step of scripts/v41_build/omlx_lattice.py:358-370
 * (nested mat-vecs, e8p_nested_m1.py:90-112) inside the layer of :327-371. */
int keep_e8_1bit_image_bytes(void);
int keep_e8_1bit_image(const uint32_t* packed_table, void* image, void* stream);
int keep_moe_layer_nested(const float* logits, const float* bias_served, const float* bias_demand,
                          int score_func, int renormalize, float route_scale, float tau,
                          const int32_t* slot_map, int64_t num_slots,
                          int64_t num_experts, int64_t k, const void* x, int x_dtype, int64_t H, int64_t I,
                          const uint16_t* gate_codes, const void* gate_scales,
                          const uint16_t* up_codes, const void* up_scales,
                          const uint16_t* down_codes, const void* down_scales, int scale_dtype,
                          int64_t group_size_h, int64_t group_size_i, const void* prepared,
                          float swiglu_limit, int32_t* idx, float* w, int32_t* want, float* want_score,
                          uint8_t* admit, void* h_work, void* out, int out_dtype,
                          const uint32_t* hot_of_slot, int64_t num_hot,
                          const uint8_t* res_gate_codes, const void* res_gate_scales,
                          const uint8_t* res_up_codes, const void* res_up_scales,
                          const uint8_t* res_down_codes, const void* res_down_scales,
                          int res_scale_dtype, int64_t res_group_size_h, int64_t res_group_size_i,
                          const void* res_image, int32_t* hot_route, void* stream);

/* Routed SwiGLU MoE for a few tokens (speculative verify) with the routes of
 * one expert sharing every code load: T tokens x k routes (idx/w [T, k], as
 * keep_moe_decode takes them), gate/up/SwiGLU into h_work ([T, k, I] bf16),
 * down per route, then out[t] = sum over the token's routes in route order of
 * w * y. Five launches on `stream` (activation terms, route plan, gate/up,
 * down, combine), no host sync. `workspace` is caller-owned device memory of
 * keep_moe_tiles_workspace_bytes(T, k, num_experts, H) bytes, 256-byte
 * aligned. The result for each token is byte-identical to keep_moe_layer's
 * for that token and routing. Replaces the layer-level use of
 * gather_vqmm_verify_rows(grouping="expert") (src/ramp/ops/vq_switch.py:
 * 286-377, tile descriptors :186-225) for the three projections and the
 * combine of deepseek_v4_flash_adapter.py:1776-1784. */
int64_t keep_moe_tiles_workspace_bytes(int64_t T, int64_t k, int64_t num_experts, int64_t H);
int keep_moe_tiles_supported(int64_t T, int64_t num_experts, int64_t H, int64_t I, int64_t k,
                             int64_t group_size_h, int64_t group_size_i);
int keep_moe_tiles(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, const int32_t* idx,
                   const float* w, int64_t k, int64_t num_experts, const uint16_t* gate_codes,
                   const void* gate_scales, const uint16_t* up_codes, const void* up_scales,
                   const uint16_t* down_codes, const void* down_scales, int scale_dtype,
                   int64_t group_size_h, int64_t group_size_i, const void* prepared,
                   float swiglu_limit, void* h_work, void* workspace, int64_t workspace_bytes,
                   void* out, int out_dtype, void* stream);

/* The few-token layer from the router logits: keep_router_dual_topk's outputs
 * (idx, w, want, want_score, admit; same contract, k <= 16) and
 * keep_moe_tiles' result, byte for byte. Up to T k = 128 routes and 512
 * experts the gate/up launch routes and plans itself (every block routes
 * every token, one wave each, plans in LDS, and forms the x terms of the
 * tiles it takes; block 0 writes the router outputs and the plan), so the
 * layer is three launches. Otherwise, for T <= 32, the router, the
 * activation terms and the route plan run as one prologue launch before
 * them (four launches); larger T runs the router and then keep_moe_tiles.
 * With slot_map
 * the pools hold num_slots rows (the plan's buckets). `workspace` holds
 * keep_moe_tiles_workspace_bytes(T, k, pool rows, H) bytes. Replaces the
 * speculative-verify decode step of scripts/v41_build/omlx_lattice.py:327-371
 * for T tokens (router :77-97, experts gather_vqmm_verify_rows
 * src/ramp/ops/vq_switch.py:286-377). */
int keep_moe_tiles_layer(const float* logits, const float* bias_served, const float* bias_demand,
                         int score_func, int renormalize, float route_scale, float tau,
                         const int32_t* slot_map, int64_t num_slots, int64_t num_experts, int64_t k,
                         const void* x, int x_dtype, int64_t T, int64_t H, int64_t I,
                         const uint16_t* gate_codes, const void* gate_scales, const uint16_t* up_codes,
                         const void* up_scales, const uint16_t* down_codes, const void* down_scales,
                         int scale_dtype, int64_t group_size_h, int64_t group_size_i, const void* prepared,
                         float swiglu_limit, int32_t* idx, float* w, int32_t* want, float* want_score,
                         uint8_t* admit, void* h_work, void* workspace, int64_t workspace_bytes, void* out,
                         int out_dtype, void* stream);

/* Prefill grouped GEMM on the fp16 matrix cores over expert-sorted routes
 * (tiles of <= 64 routes of one expert from keep_route_plan): for every tile
 * t and route i < tile_count[t], with p = tile_offset[t] + i,
 *   out[out_index[p], :] = W[tile_expert[t]] . x[lhs[p], :]
 * (lhs / out_index NULL: p itself). x is fp16, bf16 or fp32 [x_rows, K]; the
 * rows enter the matrix cores as fp16, as the reference casts them
 * (vq_switch.py:712-715,759-771): fp16 rows as they are, bf16 and fp32 rows
 * times a power of two per row (max |x| in [2^14, 2^15): no overflow, bf16
 * exact), rounded to nearest even; weights are E8P decoded exactly (x 4) from
 * T and M of `prepared` (keep_e8p_prepare), products exact, fp32 sums, scales
 * per group in fp32. `workspace` (caller-owned, 16-byte aligned) holds the
 * row factors of bf16 / fp32 input: keep_vq_grouped_gemm_q8_workspace_bytes(
 * x_rows, K) bytes (fp16 input reads none; NULL allowed). code_bits = 8
 * runs the nested tier's 8-bit E8 residual instead ([H, N, K/8] uint8 codes,
 * `prepared` = the packed 8-bit E8 table uint32[256]) and adds it to `out`,
 * which must then be fp32 (the base projection's output, e8p_nested_m1.py:
 * 90-112 run per expert tile). Replaces
 * gather_vqmm_sorted_routes' NAX E8P GEMM (src/ramp/ops/vq_switch.py:620-913;
 * native/vq_nax_ext/kernels/nax_fp16_matmul.metal:904-1062); out_index
 * folds in the scatter back to route order of
 * src/ramp/models/glm4_moe_adapter.py:274-353. */
int64_t keep_vq_grouped_gemm_q8_workspace_bytes(int64_t x_rows, int64_t K);
int keep_vq_grouped_gemm_q8(const void* x, int x_dtype, int64_t x_rows, const int32_t* lhs,
                            const int32_t* out_index, const void* codes, int code_bits, const void* scales,
                            int scale_dtype, const void* prepared, const int32_t* tile_expert,
                            const int32_t* tile_offset, const int32_t* tile_count, int64_t n_tiles,
                            int64_t routes, int64_t num_experts, int64_t N, int64_t K, int64_t group_size,
                            void* workspace, int64_t workspace_bytes, void* out, int out_dtype, void* stream);

/* The gate and up projections of the same tiles in one pass, with SwiGLU
 * (silu(min(g, L)) * clip(u, -L, L), plain for L <= 0) in fp32 and h stored
 * in bf16 at the route's sorted position: h_out[p, :] for p < routes, I
 * columns. Arithmetic and workspace as keep_vq_grouped_gemm_q8 with K = H. Replaces the
 * gate/up GEMM pair and the activation of QuantizedVQSwitchGLU's shared
 * sorted-route prefill (src/ramp/models/glm4_moe_adapter.py:274-353,355-365). */
int keep_vq_grouped_swiglu_q8(const void* x, int x_dtype, int64_t x_rows, const int32_t* lhs,
                              const uint16_t* gate_codes, const void* gate_scales, const uint16_t* up_codes,
                              const void* up_scales, int scale_dtype, const void* prepared,
                              const int32_t* tile_expert, const int32_t* tile_offset,
                              const int32_t* tile_count, int64_t n_tiles, int64_t routes, int64_t num_experts,
                              int64_t I, int64_t H, int64_t group_size, float swiglu_limit, void* workspace,
                              int64_t workspace_bytes, void* h_out, void* stream);

/* The nested 3-bit tier fused into the sorted-route prefill: as
 * keep_vq_grouped_swiglu_q8 (per-row base scales, group_size = H), and on the
 * tiles of an expert e with a residual row r = hot_row[e] (0 <= r < hot_rows;
 * -1: none) gate and up each add that row's 8-bit E8 residual,
 * R[r, n] . x * res_scale[r, n] (codes uint8 [hot_rows][I][H / 8], one scale per
 * row, res_table the packed 8-bit E8 table, uint32[256]), before the SwiGLU. A
 * hot_row entry outside [-1, hot_rows) makes that expert's h rows NaN. Replaces
 * the base GEMMs, the residual GEMMs (keep_vq_grouped_gemm_q8 with
 * code_bits = 8) and the activation of the tiered prefill, the serving
 * step's base-plus-residual (scripts/v41_build/omlx_lattice.py:172-186,
 * 358-370). */
int keep_vq_grouped_swiglu_nested_q8(const void* x, int x_dtype, int64_t x_rows, const int32_t* lhs,
                                     const uint16_t* gate_codes, const void* gate_scales, const uint16_t* up_codes,
                                     const void* up_scales, int scale_dtype, const void* prepared,
                                     const uint8_t* gate_res_codes, const void* gate_res_scales,
                                     const uint8_t* up_res_codes, const void* up_res_scales, int res_scale_dtype,
                                     const int32_t* hot_row, int64_t hot_rows, const uint32_t* res_table,
                                     const int32_t* tile_expert, const int32_t* tile_offset,
                                     const int32_t* tile_count, int64_t n_tiles, int64_t routes,
                                     int64_t num_experts, int64_t I, int64_t H, float swiglu_limit, void* workspace,
                                     int64_t workspace_bytes, void* h_out, void* stream);

/* One projection with the nested tier fused in (the down projection of the
 * tiered prefill): keep_vq_grouped_gemm_q8 on E8P codes with per-row scales
 * (group_size = K), plus, on the tiles of a hot expert, its residual row's
 * 8-bit E8 codes (uint8 [hot_rows][N][K / 8], one scale per row), added before
 * the store. hot_row and res_table as keep_vq_grouped_swiglu_nested_q8.
 * Replaces the tiered prefill's base GEMM plus residual GEMM of one projection
 * (scripts/v41_build/omlx_lattice.py:172-186). */
int keep_vq_grouped_gemm_nested_q8(const void* x, int x_dtype, int64_t x_rows, const int32_t* lhs,
                                   const int32_t* out_index, const uint16_t* codes, const void* scales,
                                   int scale_dtype, const void* prepared, const uint8_t* res_codes,
                                   const void* res_scales, int res_scale_dtype, const int32_t* hot_row,
                                   int64_t hot_rows, const uint32_t* res_table, const int32_t* tile_expert,
                                   const int32_t* tile_offset, const int32_t* tile_count, int64_t n_tiles,
                                   int64_t routes, int64_t num_experts, int64_t N, int64_t K, void* workspace,
                                   int64_t workspace_bytes, void* out, int out_dtype, void* stream);

/* Weighted combine of per-route outputs: out[t, :] = sum over j < k, in
 * order, of w[t, j] * y[t k + j, :] with fp32 multiply-adds (a NaN route row
 * stays NaN whatever its weight). y fp32 [T k, H], w fp32 [T, k]. Replaces the
 * MoE block's (y * scores[..., None]).sum(axis=-2)
 * (src/ramp/models/glm4_moe_adapter.py:367-372). */
int keep_route_combine(const float* y, const float* w, int64_t T, int64_t k, int64_t H, void* out, int out_dtype,
                       void* stream);

/* Random-sign Walsh-Hadamard transform of T rows of n activations (16 <= n <= 8192,
 * a power of two): forward y = FWHT(x * signs) / sqrt(n), inverse (inverse != 0)
 * y = (FWHT(x) / sqrt(n)) * signs; signs = NULL applies the plain orthonormal FWHT.
 * float32 butterflies in the reference's stage order, so float32 output is
 * bit-identical to apply_rht_np / apply_inverse_rht_np. x and signs 16-byte
 * aligned, out a separate buffer. n outside the served range -> KEEP_EUNSUPPORTED.
 * Replaces apply_rht_np src/keep/quant/rht.py:51-57, apply_inverse_rht_np :60-66,
 * apply_rht_mx :84-91 (as applied in src/ramp/nn/switch_linear.py:320-322). */
int keep_rht(const void* x, int x_dtype, const float* signs, int inverse, int64_t T, int64_t n, void* out,
             int out_dtype, void* stream);

/* The steps in front of the routed experts, one row pass per token (rows of
 * n = 64..8192 values, a power of two):
 *   y = round_x(gamma * (x / sqrt(mean(x^2) + eps)))   RMSNorm in fp32, rounded to
 *       x's dtype (gamma NULL: 1); written to `normed` (x's dtype) when non-null
 *       (the router's input);
 *   q = round_x(e4m3(clamp(y / s, +-448)) * s) per quant_block values, s =
 *       max(amax, 1e-4) / 448, rounded up to a power of two when pow2_scales,
 *       e4m3 = nearest FP8 e4m3fn value, ties to even (quant_block 0: q = y);
 *   out = RHT(q, signs) as keep_rht (signs NULL: out = q), in out_dtype.
 * Replaces the expert-input preparation of the serving step: ffn_norm
 * (src/ramp/models/deepseek_v4_flash_adapter.py:1792-1807), act_quant
 * (scripts/runpod/v41_reap/torch_kernel.py:40-53, used at
 * scripts/v41_build/omlx_lattice.py:332,357) and apply_rht_mx
 * (src/keep/quant/rht.py:84-91). */
int keep_rmsnorm_quant_rht(const void* x, int x_dtype, int64_t T, int64_t n, const void* gamma,
                           int gamma_dtype, float eps, int64_t quant_block, int pow2_scales,
                           const float* signs, void* normed, void* out, int out_dtype, void* stream);

/* After the routed combine: out[i] = round_out(residual[i] + (routed[i] +
 * shared[i])) over n values, fp32 sums in that order (shared and residual
 * optional, any dtype; out may alias routed or residual). The MoE's routed sum
 * plus the shared expert (src/ramp/models/deepseek_v4_flash_adapter.py:1784;
 * the serving step's shared down adds the fp32 routed sum and rounds to bf16,
 * scripts/v41_build/omlx_lattice.py:374-388), with the block's residual add. */
int keep_moe_combine_add(const float* routed, const void* shared, int shared_dtype, const void* residual,
                         int residual_dtype, int64_t n, void* out, int out_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KEEP_AMD_H */
