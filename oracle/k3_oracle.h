/* CPU oracle for the K3 prefill memory-bound op family.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: it is loaded by the
 * tests, by __graft_entry__.smoke() and by the CPU-baseline leg of bench.py,
 * never by the product path (kern-k3_amd/), which runs only on the GPU.
 *
 * Each function restates the arithmetic of a reference kernel in plain C,
 * citing the reference file:line it follows.  Floating-point operations are
 * single IEEE f32 operations (compiled with -ffp-contract=off); a fused
 * multiply-add appears only as an explicit fmaf, where the reference's
 * compiler contracts `a += x * y`.  Reductions replay the reference's order
 * (per-thread serial sums, 32-lane xor butterflies, fixed-order partials).
 *
 * Where the reference calls an approximate CUDA intrinsic, the oracle uses a
 * correctly rounded or documented replacement, named in the function's
 * comment:
 *   rsqrtf(v)      -> 1.0f / sqrtf(v), both correctly rounded;
 *   expf / __expf  -> k3o_expf, a Cody-Waite + degree-7 Taylor exp whose
 *                     steps are all correctly rounded f32 operations;
 *   e4m3 / bf16    -> exact OCP / IEEE round-to-nearest-even encoders.
 *
 * bf16 tensors are uint16_t bit patterns; e4m3 and E8M0 tensors are uint8_t.
 */
#ifndef K3_ORACLE_H
#define K3_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- numerics ---------------------------------------------------------- */
float k3o_bf2f(uint16_t h);
uint16_t k3o_f2bf(float f);
uint8_t k3o_e4m3(float x);
float k3o_e4m3_decode(uint8_t c);
float k3o_expf(float x);
float k3o_sigmoid(float x);
int k3o_mx_exp(float amax);
void k3o_f2bf_n(const float* x, uint16_t* y, size_t n);
void k3o_e4m3_n(const float* x, uint8_t* y, size_t n);
void k3o_expf_n(const float* x, float* y, size_t n);

/* ---- K1 residual family (k3_residual_v2.cu) ---------------------------- */
/* partial_bf16 or partial_f32 (exactly one non-null) selects LAND_BF16. */
void k3o_land_add_attnres_rms(const uint16_t* partial_bf16, const float* partial_f32,
                              const uint16_t* prefix, const uint16_t* blocks,
                              const float* sw, const uint16_t* gamma, uint16_t* prefix2,
                              uint16_t* normed, int nb, int snapshot, int B, float eps);
void k3o_attnres_rms(const uint16_t* prefix, uint16_t* blocks, const float* sw,
                     const uint16_t* gamma, uint16_t* normed, int nb, int snapshot, int B,
                     float eps);
void k3o_land_add2(const float* p1, const float* p2, const uint16_t* prefix2, uint16_t* hidden,
                   int two, int B);
/* statistics hand-off res_in -> res_mlp (k3_residual_push_stats.cu,
 * k3_residual_nb_stats.cu); stats are [B, 8, 2] f32 */
void k3o_attnres_rms_stats(const uint16_t* prefix, uint16_t* blocks, const float* sw,
                           const uint16_t* gamma, uint16_t* normed, int nb, int snapshot, int B,
                           float eps, const float* sw_mlp, float* stats);
void k3o_land_add_attnres_rms_stats(const uint16_t* partial_bf16, const float* partial_f32,
                                    const uint16_t* prefix, const uint16_t* blocks,
                                    const float* sw, const uint16_t* gamma, uint16_t* prefix2,
                                    uint16_t* normed, int nb, int snapshot, int B, float eps,
                                    const float* stats, int nb_stats);
void k3o_land_add2_bf16(const uint16_t* p1, const uint16_t* p2, const uint16_t* prefix2,
                        uint16_t* hidden, int two, int B);

/* ---- MXFP8 (k3_moe_prefill_v4.cu:111-140) and the fused op ------------- */
void k3o_moe_quant(const uint16_t* x, uint8_t* q, uint8_t* sf, int rows, int cols);
void k3o_residual_rms_mxfp8(const uint16_t* x, const uint16_t* residual, const uint16_t* gamma,
                            uint16_t* residual_out, uint8_t* q, uint8_t* sf, uint16_t* normed,
                            int B, float eps);

/* ---- per-tensor fp8 pair (k3_quant_fp8_pair{,_v2}.cu) ------------------- */
void k3o_quant_fp8_amax(const uint16_t* x, int n, float* partials, int nb_grid, int v2);
void k3o_quant_fp8_apply(const uint16_t* x, uint8_t* y, int n, const float* partials, int nb,
                         float* scale_out);

/* ---- router / argmax (k3_router_argmax.cu) ------------------------------ */
uint32_t k3o_ord_f32(float f);
void k3o_sigmoid_n(const float* x, float* y, size_t n);
void k3o_router_topk(const float* S, const float* bias, const uint16_t* rs, int* idx, float* wts,
                     int B, int topk);
void k3o_argmax_partial(const float* logits, float* pmax, int* pidx, int B, int n, int parts);
void k3o_argmax_final(const float* pmax, const int* pidx, long long* out, int B, int parts);

/* ---- EP routing, permute, finalize, weight layouts (k3_moe_prefill_v4.cu) -- */
int k3o_local_expert(int id, int rank, int E, int ep_ranks, int strided);
void k3o_route_count(const int* ids, int T, int topk, int rank, int E, int ep_ranks, int strided,
                     int* blockcount);
void k3o_route_tables(const int* blockcount, int blocks, int E, int tile, int* blockoff,
                      int* cta_batch, int* cta_limit, int* num_non_exiting, int* total_padded,
                      int* route_map);
void k3o_route_scatter(const int* ids, const int* blockoff, int T, int topk, int rank, int E,
                       int ep_ranks, int strided, int* route_map, int* exp2perm);
void k3o_moe_permute_mx(const uint8_t* q, const uint8_t* sf, const int* route_map,
                        int total_padded, int cols, uint8_t* pq, uint8_t* psf);
void k3o_moe_finalize(const uint16_t* fc2, const int* exp2perm, const float* wts, uint16_t* out,
                      int T, int topk, int cols);
void k3o_moe_w_shuffle(const uint8_t* src, uint8_t* dst, int experts, int n, int row_bytes,
                       int gated);
void k3o_moe_sf_shuffle(const uint8_t* src, uint8_t* dst, int experts, int n, int kg, int gated);

/* ---- KDA span gather / output gate (k3_span_gather_v3.cu, k3_kda_out_gate_v3.cu) */
void k3o_span_gather(const uint16_t* partial, const float* cw, uint16_t* win, const float* wsm,
                     uint16_t* span_q, uint16_t* span_k, uint16_t* span_v, uint16_t* span_beta,
                     uint16_t* span_flow, int at, int span, int heads);
void k3o_kda_out_gate(const uint16_t* attn, const uint16_t* gate_partial, const float* gamma_o,
                      uint16_t* gated, int at, int span, int heads, float eps);

/* ---- MLA (k3_mla_prep_v2.cu / k3_mla_prep_bf16.cu; RoPE + pack) -------------- */
void k3o_mla_prep(const float* partial_f32, const uint16_t* partial_bf16, int mla_fused,
                  int inner, const uint16_t* gamma_q_a, const uint16_t* gamma_kv_a,
                  const long long* slot_mapping, uint16_t* slab, long long layer_off,
                  long long page_stride, uint16_t* q_norm, uint16_t* mla_gate, int B);
void k3o_mla_rope_pack(const uint16_t* latent, const uint16_t* k_rope, const uint16_t* q,
                       const uint16_t* gamma_kv, const long long* positions, uint16_t* latent_out,
                       uint16_t* q_out, float theta, float eps, int T, int H);

/* ---- landing kernels (k3_land.cu, k3_land_bf16.cu, k3_situ_bf16.cu, k3_land_fused.cu) */
void k3o_rms(const uint16_t* x, const uint16_t* gamma, uint16_t* o, int h, int B);
void k3o_land(const float* p, uint16_t* o, int n, int off, int ldc, int B);
float k3o_situ(float g, float u);
void k3o_situ_n(const float* g, const float* u, float* y, size_t n);
/* exactly one of p_f32 / p_bf16 is non-null */
void k3o_land_situ(const float* p_f32, const uint16_t* p_bf16, uint16_t* act, int n, int B);
void k3o_situ_rms(const uint16_t* sp, uint16_t* act, const uint16_t* lat, const uint16_t* gam,
                  uint16_t* ln, int n, int B, int h, int L, int tokens);

int k3o_num_threads(void);
void k3o_par_copy(void* dst, const void* src, size_t n);

/* ---- MoE expert GEMMs (k3_oracle_gemm.c) */
float k3o_e2m1_decode(uint8_t nib);
void k3o_moe_gemm_mx(const uint8_t* a, const uint8_t* a_sf, const int* a_rows, const uint8_t* w,
                     const uint8_t* w_sf, int num_tiles, const int* cta_batch, int E, int N, int K,
                     double* out);
void k3o_moe_gemm_mx_abs(const uint8_t* a, const uint8_t* a_sf, const int* a_rows,
                         const uint8_t* w, const uint8_t* w_sf, int num_tiles,
                         const int* cta_batch, int E, int N, int K, double* out);
void k3o_situ_ab_n(const float* g, const float* u, float* y, size_t n, float alpha, float beta);

/* ---- epoch / arrival barrier for host threads (k3_oracle_barrier.c) */
void k3o_flags_init(uint64_t* flags, int n);
void k3o_epoch_bump(uint64_t* flags, int units);
unsigned k3o_rs_arrive(uint64_t* flags, const uint64_t* flags_peer, int units, int slot,
                       int nranks, long long spin_ns);

#ifdef __cplusplus
}
#endif
#endif
