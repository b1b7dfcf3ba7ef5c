/* k3h: C-ABI for the MI355X (gfx950) K3 prefill memory-bound op family.
 *
 * Two layers:
 *
 * 1. Module layer -- the drop-in for the kern runtime's cubin loading.  The
 *    reference runtime loads one code object per module key (kernels.toml:66-76,
 *    126-135, 203-230, 243-253) and launches `extern "C"` entries with a packed
 *    parameter buffer laid out at natural alignment (pointers / i64 at 8 bytes,
 *    i32 / f32 at 4), grid and block from the manifest's launch description
 *    (manifest ops.<op>.impl.launches, e.g. k3-tp4-prefill-16k.json:404788).
 *    k3h_module_* / k3h_function / k3h_launch do the same over hipModule with
 *    gfx950 code objects that export the same entry names.
 *
 * 2. Operator layer -- one typed wrapper per hot manifest op, computing grid and
 *    block exactly as the manifest's grid expressions do, validating arguments
 *    on the host, and launching on the caller's stream.
 *
 * Conventions: every function returns K3H_OK (0) or a negative code; a HIP
 * error e is returned as K3H_EHIP_BASE - e.  No exceptions cross the ABI.
 * Streams are hipStream_t passed as void* (NULL = the default stream).  Device
 * pointers are plain pointers; bf16 tensors are 16-bit patterns, e4m3 / E8M0
 * tensors bytes.  Launches are stream-ordered, allocate nothing and are
 * graph-capturable.  Module handles are immutable after load; a context
 * serialises its lazy module loads internally and may be shared by threads.
 */
#ifndef K3H_H
#define K3H_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define K3H_API __attribute__((visibility("default")))

#define K3H_OK 0
#define K3H_EINVAL (-1)    /* bad argument: null/misaligned pointer, size, range */
#define K3H_ENOMODULE (-2) /* code object missing or not loadable */
#define K3H_ENOENTRY (-3)  /* entry name not in the module */
#define K3H_ENOMEM (-4)
#define K3H_ERESIDENT (-5) /* the device cannot hold a grid-synchronised launch at once */
#define K3H_EHIP_BASE (-1000)

typedef struct k3h_module_s* k3h_module_t;
typedef struct k3h_fn_s* k3h_fn_t;
typedef struct k3h_ctx_s* k3h_ctx_t;

/* ---- module layer --------------------------------------------------------
 * Replaces the kern runtime's cubin load / entry lookup / launch (README.md:92-97
 * of the reference; manifest `modules` and `impl.launches`). */
K3H_API int k3h_module_load(const void* image, size_t bytes, k3h_module_t* out);
K3H_API int k3h_module_load_file(const char* path, k3h_module_t* out);
K3H_API int k3h_function(k3h_module_t mod, const char* entry, k3h_fn_t* out);
K3H_API int k3h_launch(k3h_fn_t fn, const uint32_t grid[3], const uint32_t block[3],
                       uint32_t shmem, void* stream, const void* packed_args, size_t bytes);
K3H_API int k3h_module_unload(k3h_module_t mod);
K3H_API const char* k3h_error_string(int code);
/* HIP runtime version the library is bound to (hipRuntimeGetVersion). */
K3H_API int k3h_runtime_version(int* version);

/* ---- context: code objects by module key ---------------------------------
 * <dir>/<module key>.hsaco, loaded on first use (e.g. "k3_residual_v2+LAND_BF16=1")
 * into the device current at that moment: use one context per device. */
K3H_API int k3h_ctx_create(const char* codeobj_dir, k3h_ctx_t* out);
K3H_API int k3h_ctx_destroy(k3h_ctx_t ctx);
K3H_API int k3h_ctx_function(k3h_ctx_t ctx, const char* module_key, const char* entry,
                             k3h_fn_t* out);

/* ---- K1 residual family ---------------------------------------------------
 * eps selects the code object: 1e-5 (the reference's compiled KEPS,
 * k3_residual_v2.cu:54) or 1e-6 (the "+K3_EPS=1e-6f" build); others: K3H_EINVAL. */

/* kern_k3_land_add_attnres_rms (k3_residual_v2.cu:295; manifest op
 * land_add_attnres_rms_bf16_v2, l0-bf16 json:401328).  grid (B), block 128.
 * land_bf16 != 0: partial is bf16 [B,7168] (module +LAND_BF16=1), else f32. */
K3H_API int k3h_land_add_attnres_rms(k3h_ctx_t ctx, void* stream, int land_bf16,
                                     const void* partial, const void* prefix,
                                     const void* blocks, const float* sw, const void* gamma,
                                     void* prefix2, void* normed, int nb, int snapshot, int B,
                                     float eps);
/* kern_k3_land_add_attnres_rms_nb{1..8} (k3_residual_nb.cu:350-811; manifest op
 * land_add_attnres_rms_bf16_v2_nb1, json:406888).  LAND_BF16 only; 1 <= nb <= 8. */
K3H_API int k3h_land_add_attnres_rms_nb(k3h_ctx_t ctx, void* stream, const void* partial,
                                        const void* prefix, const void* blocks, const float* sw,
                                        const void* gamma, void* prefix2, void* normed, int nb,
                                        int snapshot, int B);
/* kern_k3_attnres_rms (k3_residual_v2.cu:260; op attnres_rms_v2, l0-bf16 json:401191). */
K3H_API int k3h_attnres_rms(k3h_ctx_t ctx, void* stream, const void* prefix, void* blocks,
                            const float* sw, const void* gamma, void* normed, int nb,
                            int snapshot, int B, float eps);
/* kern_k3_land_add2 (k3_residual_v2.cu:349; op land_add2_v2, l0-bf16 json:401295). */
K3H_API int k3h_land_add2(k3h_ctx_t ctx, void* stream, const float* p1, const float* p2,
                          const void* prefix2, void* hidden, int two, int B);

/* ---- residual push family (res_in / res_mlp of the TP4 prefill) -------------
 * kern_k3_attnres_rms_push: K1a's row body whose normed row b lands at row
 * rank*B + b of every rank's normed_all [nranks*B, 7168]: the local copy via
 * normed_all, rank q != rank via dst_peer[q] (u64 device addresses, nranks <= 8;
 * on one GPU they may all be local buffers).  grid (B), block 128, eps 1e-5.
 *   version 1 / 3: modules k3_residual_push / k3_residual_push_v3
 *     (k3_residual_push.cu:320, k3_residual_push_v3.cu:324; manifest op
 *     attnres_rms_push_first_v3, k3-tp4-prefill-16k.json:406806);
 *   k3h_attnres_rms_push_stats: module k3_residual_push_stats
 *     (k3_residual_push_stats.cu:354): also stats [B,8,2] f32 = (sum x^2,
 *     sum x*sw_mlp) of block candidates c < nb;
 *   k3h_attnres_rms_push_add2: module k3_residual_push_add2
 *     (k3_residual_push_add2.cu:362; op attnres_rms_push_add2, json:407299): the
 *     prefix row is hidden = bf16(prefix2 + p1 [+ p2]) (bf16 inputs), also stored. */
K3H_API int k3h_attnres_rms_push(k3h_ctx_t ctx, void* stream, int version, const void* prefix,
                                 void* blocks, const float* sw, const void* gamma,
                                 void* normed_all, const unsigned long long* dst_peer, int nb,
                                 int snapshot, int B, int rank, int nranks);
K3H_API int k3h_attnres_rms_push_stats(k3h_ctx_t ctx, void* stream, const void* prefix,
                                       void* blocks, const float* sw, const void* gamma,
                                       void* normed_all, const unsigned long long* dst_peer,
                                       int nb, int snapshot, int B, int rank, int nranks,
                                       const float* sw_mlp, float* stats);
K3H_API int k3h_attnres_rms_push_add2(k3h_ctx_t ctx, void* stream, void* blocks, const float* sw,
                                      const void* gamma, void* normed_all,
                                      const unsigned long long* dst_peer, int nb, int snapshot,
                                      int B, int rank, int nranks, const float* sw_mlp,
                                      float* stats, const void* p1, const void* p2,
                                      const void* prefix2, void* hidden, int two);
/* kern_k3_land_add_attnres_rms_nb{1..8} of module k3_residual_nb_stats (LAND_BF16)
 * (k3_residual_nb_stats.cu:366-811; ops land_add_attnres_rms_bf16_v2_nb4..8,
 * json:406999): as k3h_land_add_attnres_rms_nb, with candidates c < nb_stats
 * (0 <= nb_stats <= nb) scored from stats [B,8,2] written by res_in. */
K3H_API int k3h_land_add_attnres_rms_nb_stats(k3h_ctx_t ctx, void* stream, const void* partial,
                                              const void* prefix, const void* blocks,
                                              const float* sw, const void* gamma, void* prefix2,
                                              void* normed, int nb, int snapshot, int B,
                                              const float* stats, int nb_stats);
/* kern_k3_land_add2_bf16 (k3_land_bf16.cu:96; module k3_land_bf16): K1c with
 * bf16 partials.  grid (B, 1), block 128. */
K3H_API int k3h_land_add2_bf16(k3h_ctx_t ctx, void* stream, const void* p1, const void* p2,
                               const void* prefix2, void* hidden, int two, int B);

/* ---- epoch / arrival barrier of the push family ------------------------------
 * flags: this rank's u64 counters (the manifest's coll_flags [372]); flags[0] is
 * the epoch.  flags_peer: u64 device addresses of every rank's flags, rank q at
 * [q] (the manifest's coll_flags_peer).  Counters are never reset after init.
 * kern_k3_flags_init (k3_collectives.cu:64; op k3_flags_init of the load program,
 * k3-tp4-prefill-16k.json:406338): flags[0 .. n) = 0.  Grid 1, block 256. */
K3H_API int k3h_flags_init(k3h_ctx_t ctx, void* stream, unsigned long long* flags, int n);
/* kern_k3_epoch_bump (k3_collectives.cu:74; op k3_epoch_bump, the first call of
 * every prefill, json:406299): flags[0] += units, the arrivals the call's
 * collectives will add per slot (the collective grid: 896 at 16,384 tokens).
 * Grid (units), block 64: the entry adds its grid size. */
K3H_API int k3h_epoch_bump(k3h_ctx_t ctx, void* stream, unsigned long long* flags, int units);
/* kern_k3_rs_arrive1 (k3_rs_arrive_v2.cu:41; module k3_rs_arrive_v2 of op
 * k3_allgather_push, json:406354, the normed_sync after every residual push, and
 * the first launch of k3_reducescatter_bf16, json:406431): flags[slot] += units,
 * then wait until every rank q < nranks has flags_peer[q][slot] >= flags[0]
 * (low 32 bits compared), giving up after 2 s per rank.  1 <= slot, 1 <= nranks
 * <= 8.  Grid 1, block 64.  missing == NULL launches the manifest entry; else the
 * entry k3h_rs_arrive_mask (no counterpart in the reference) runs the same
 * barrier and writes *missing (device u32) = mask of the ranks that had not
 * arrived when the wait gave up, 0 when all did. */
K3H_API int k3h_rs_arrive(k3h_ctx_t ctx, void* stream, unsigned long long* flags,
                          const unsigned long long* flags_peer, int units, int slot, int nranks,
                          unsigned* missing);

/* ---- landing kernels (shared-expert MLP, MoE latent norm) -------------------
 * The entries run under the manifests' grids; these typed calls launch compact
 * grids of 256-thread blocks sized to the work where the shape allows (the
 * manifest grids' idle waves cost more than the work on MI355X).
 * kern_k3_rms (k3_land.cu:104; l0-bf16 op rms, json:399525): o = bf16(x * r) (x)
 * gamma, r = 1/sqrt(sum x^2 / h + 1e-5); x, o [B, h] bf16.  Manifest grid (B),
 * block 1024; typed call ceil(B/4) x 256 when h % 8 == 0 and h <= 8192. */
K3H_API int k3h_rms(k3h_ctx_t ctx, void* stream, const void* x, const void* gamma, void* o, int h,
                    int B);
/* kern_k3_land (k3_land.cu:168; l0-bf16 op land_n3584, json:400710):
 * o[b, i] = bf16(p[b*ldc + off + i]), i < n.  Manifest grid (B, ceil(n/1024)),
 * block 1024; typed call ceil(B*n/2048) x 256 when (n | off | ldc) % 4 == 0. */
K3H_API int k3h_land(k3h_ctx_t ctx, void* stream, const float* p, void* o, int n, int off, int ldc,
                     int B);
/* SiTU landing act[b, i] = bf16(4 tanh(g/4) sigmoid(g) * 25 tanh(u/25)), gate g and
 * up u the two halves of row b of p [B, 2n] (landed to bf16 first).  bf16_in:
 *   0  kern_k3_land_situ, p f32 (k3_land.cu:211; op land_situ_n33792,
 *      k3-tp4-prefill-16k.json:405746; l0 op land_situ_n6144, json:400768);
 *   1  kern_k3_land_situ_bf16, p bf16 (k3_land_bf16.cu:56; module k3_land_bf16);
 *   2  kern_k3_situ_bf16, p bf16 (k3_situ_bf16.cu:9; l0 op land_situ_n33792,
 *      json:400660).
 * Manifest grid (B, ceil(n/1024)), block 1024; typed call ceil(B*n/2048) x 256
 * when n % 8 == 0. */
K3H_API int k3h_land_situ(k3h_ctx_t ctx, void* stream, int bf16_in, const void* p, void* act,
                          int n, int B);
/* kern_k3_situ_rms_bf16 (k3_land_fused.cu:151; op land_situ_rms, json:406727): the
 * bf16 SiTU landing of sp [B, 2n] -> act [B, n] and the rms of lat [L, h] -> ln
 * in one launch.  grid 3 ceil(tokens/16), block 512; needs 4 ceil(tokens/16) >= B, L. */
K3H_API int k3h_situ_rms(k3h_ctx_t ctx, void* stream, const void* sp, void* act, const void* lat,
                         const void* gam, void* ln, int n, int B, int h, int L, int tokens);

/* ---- MXFP8 -----------------------------------------------------------------
 * kern_k3_moe_quant (k3_moe_prefill_v4.cu:111; manifest op moe_quant, json:404926).
 * grid ceil(rows*cols/32/256), block 256; rows*cols % 32 == 0. */
K3H_API int k3h_moe_quant(k3h_ctx_t ctx, void* stream, const void* x, void* q, void* sf,
                          int rows, int cols);

/* ---- per-tensor fp8 pair ---------------------------------------------------
 * kern_quant_fp8_amax[_v2] + kern_quant_fp8_apply[_v2] (k3_quant_fp8_pair.cu:18,32;
 * k3_quant_fp8_pair_v2.cu:42,63; manifest op quant_fp8_tensor, json:407194):
 * partials[nb] f32 (scratch owned by the caller), scale_out[1] f32, y u8 [n].
 * Both launches grid (nb), block 256; the manifest uses nb = 2048.  v2 != 0
 * selects the _v2 module.  The amax and apply steps are also exported alone. */
K3H_API int k3h_quant_fp8_amax(k3h_ctx_t ctx, void* stream, int v2, const void* x, int n,
                               float* partials, int nb);
K3H_API int k3h_quant_fp8_apply(k3h_ctx_t ctx, void* stream, int v2, const void* x, void* y,
                                int n, const float* partials, int nb, float* scale_out);
K3H_API int k3h_quant_fp8_tensor(k3h_ctx_t ctx, void* stream, int v2, const void* x, void* y,
                                 float* scale_out, float* partials, int n, int nb);
/* k3h_quant_fp8_tensor_noalloc: no counterpart in the reference.  For callers
 * that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): k3h_quant_fp8_tensor with the nb amax
 * partials in a device array of this library (K3H_NOALLOC_MAX_NB floats, one
 * copy per GPU, held until the process ends) instead of a caller buffer.  nb
 * above K3H_NOALLOC_MAX_NB is K3H_EINVAL.  The first call on a device resolves
 * the array's address (and, like every entry, loads the code object on first
 * use); no call allocates device memory.  Every call on one GPU shares the
 * array: calls that overlap on one GPU race and must be serialised. */
#define K3H_NOALLOC_MAX_NB 4096
K3H_API int k3h_quant_fp8_tensor_noalloc(k3h_ctx_t ctx, void* stream, int v2, const void* x,
                                         void* y, float* scale_out, int n, int nb);

/* k3h_residual_rms_mxfp8: fused residual add + RMSNorm + MXFP8 (no single
 * reference entry: K1b at nb = 0 composed with kern_k3_moe_quant).  Module
 * k3h_fused; grid ceil(B/2), block 256 (two rows per workgroup).  normed may be
 * NULL; sf must be 4-byte aligned. */
K3H_API int k3h_residual_rms_mxfp8(k3h_ctx_t ctx, void* stream, const void* x,
                                   const void* residual, const void* gamma, void* residual_out,
                                   void* q, void* sf, void* normed, float eps, int B);

/* ---- MoE router (module k3_router_argmax[+TOPK=8]) ----------------------------
 * kern_k3_router_topk (k3_router_argmax.cu:87; manifest op router_topk,
 * json:404788): S f32 [B,224], bias f32 [224], rs bf16 [1] -> idx i32 [B,topk],
 * wts f32 [B,topk].  grid (B), block 256.  topk 16 (manifest) or 8. */
K3H_API int k3h_router_topk(k3h_ctx_t ctx, void* stream, int topk, const float* S,
                            const float* bias, const void* rs, int* idx, float* wts, int B);
/* kern_k3_argmax_f32_partial + _final (k3_router_argmax.cu:186,227; op
 * argmax_f32_one): pmax/pidx [B*parts] scratch, out i64 [B]. */
K3H_API int k3h_argmax_f32(k3h_ctx_t ctx, void* stream, const float* logits, float* pmax,
                           int* pidx, long long* out, int B, int n, int parts);

/* ---- EP routing (module k3_moe_prefill_v4+EP_RANKS=4+EP_STRIDED=1+TILE_SHIFT=7+
 * SCATTER_WARPS=16[+TOPK=8]); experts placed strided: id % 4 == rank -> id / 4. */
/* kern_k3_moe_route_count (k3_moe_prefill_v4.cu:142; op moe_route_count,
 * json:404991): ids i32 [T,topk] -> blockcount i32 [ceil(T/256), E]. */
K3H_API int k3h_moe_route_count(k3h_ctx_t ctx, void* stream, int topk, const int* ids, int T,
                                int rank, int E, int* blockcount);
/* kern_k3_moe_route_tables (k3_moe_prefill_v4.cu:159; op moe_route_tables,
 * json:405046).  grid 1, block 1024; tile must be 128. */
K3H_API int k3h_moe_route_tables(k3h_ctx_t ctx, void* stream, const int* blockcount, int blocks,
                                 int E, int tile, int* blockoff, int* cta_batch, int* cta_limit,
                                 int* num_non_exiting, int* total_padded, int* route_map);
/* kern_k3_moe_route_scatter (k3_moe_prefill_v4.cu:205; op moe_route_scatter,
 * json:405120): route_map i32 [total_padded] (inout), exp2perm i32 [T,topk]. */
K3H_API int k3h_moe_route_scatter(k3h_ctx_t ctx, void* stream, int topk, const int* ids,
                                  const int* blockoff, int T, int rank, int E, int* route_map,
                                  int* exp2perm);
/* k3h_moe_route: no reference entry (the reference runs route_count,
 * route_tables and route_scatter as three launches).  The same outputs as that
 * chain -- blockcount, blockoff, cta_batch, cta_limit, num_non_exiting,
 * total_padded, route_map, exp2perm, bit for bit -- from one launch of
 * k3h_moe_route_fused (module k3_moe_prefill_v4+...[+TOPK=8]; grid
 * ceil(T / 256) <= 256, i.e. T <= 65536, block 512), whose workgroups meet at
 * one grid barrier.  sync: 2 ints of device memory, zero before the first call;
 * each call leaves them zero again.  Calls that share `sync` must not overlap
 * (stream-order them).  Before launching, the call checks that the device holds
 * the whole grid at once (occupancy x CUs, cached per context and device) and
 * returns K3H_ERESIDENT otherwise.  The barrier's wait is still bounded and
 * all-or-nothing: if it expires (some workgroup never became resident) no
 * workgroup proceeds, num_non_exiting = 0, total_padded = -1 and every
 * exp2perm entry is -1 (nothing routed: the GEMMs and the permute see no tile,
 * finalize no local slot); blockoff, cta_batch, cta_limit and route_map are
 * then not written, and `sync` still comes back zero.  T = 0 writes
 * num_non_exiting = total_padded = 0. */
K3H_API int k3h_moe_route(k3h_ctx_t ctx, void* stream, int topk, const int* ids, int T, int rank,
                          int E, int* blockcount, int* blockoff, int* cta_batch, int* cta_limit,
                          int* num_non_exiting, int* total_padded, int* route_map, int* exp2perm,
                          int* sync);
/* kern_k3_moe_finalize (k3_moe_prefill_v4.cu:254; op moe_finalize, json:405686):
 * fc2 bf16 [total_padded, cols], wts f32 [T,topk] -> out bf16 [T, cols];
 * cols % 8 == 0.  The manifest entry runs grid ceil(T/2), block 128 (one wave per
 * token); this call launches k3h_moe_finalize_rows of the same module, grid T,
 * block 448 (one workgroup per token), whose outputs are the same bits. */
K3H_API int k3h_moe_finalize(k3h_ctx_t ctx, void* stream, int topk, const void* fc2,
                             const int* exp2perm, const float* wts, void* out, int T, int cols);
/* k3h_moe_permute_mx: no reference entry (moe_fc1 gathers through route_map
 * inside the GEMM, ops.moe_fc1 json:405185).  pq[r] = q[route_map[r]] (cols
 * e4m3 bytes), psf[r] = sf[route_map[r]] (cols/32 E8M0 bytes) for
 * r < min(*total_padded, max_rows); *total_padded is a device value and pq / psf
 * hold max_rows rows (size them by the route_map capacity, T*topk + E*127, to
 * cover every routing).  Grid ceil(max_rows/4) x 256; cols % 1024 == 0, <= 16384. */
K3H_API int k3h_moe_permute_mx(k3h_ctx_t ctx, void* stream, const void* q, const void* sf,
                               const int* route_map, const int* total_padded, int max_rows,
                               int cols, void* pq, void* psf);
/* kern_k3_moe_w_shuffle / kern_k3_moe_sf_shuffle (k3_moe_prefill_v4.cu:310,320):
 * load-time weight / scale layouts of the grouped GEMM. */
K3H_API int k3h_moe_w_shuffle(k3h_ctx_t ctx, void* stream, const void* src, void* dst,
                              int experts, int n, int row_bytes, int gated);
K3H_API int k3h_moe_sf_shuffle(k3h_ctx_t ctx, void* stream, const void* src, void* dst,
                               int experts, int n, int kg, int gated);

/* ---- KDA (modules k3_span_gather_v3+HEADS=24, k3_kda_out_gate_v3+HEADS=24) ----
 * kern_k3_span_gather (k3_span_gather_v3.cu:251; op span_gather_v2, json:406197):
 * partial bf16 [rows, 4*3072] (q|k|v|g bands), cw f32 [3][4][3072], kda_base:
 * the KDA state (windows at line_index[at]*line_bytes + 24*128*128*4 + s*18432),
 * wsm_partial f32 [rows, 256] -> span_q/k/v bf16 [span, 3072], span_beta bf16
 * [24*span], span_flow bf16 [span, 128].  span_at: device i32 [1]. */
K3H_API int k3h_span_gather(k3h_ctx_t ctx, void* stream, const void* partial, const float* cw,
                            void* kda_base, const int* line_index, long long line_bytes,
                            const float* wsm_partial, void* span_q, void* span_k, void* span_v,
                            void* span_beta, void* span_flow, const int* span_at, int span);
/* kern_k3_kda_out_gate (k3_kda_out_gate_v3.cu:36; op kda_out_gate_v2,
 * json:406169): attn bf16 [span, 3072], gate band 3 of gate_partial bf16
 * [rows, 12288], gamma_o f32 [128] -> gated bf16 rows [at, at + span).
 * eps is the per-head RMSNorm eps, compiled into the module as the reference's
 * define (k3_kda_out_gate_v3.cu:25): 1e-5f (k3_kda_out_gate_v3+HEADS=24) or
 * 1e-6f (k3_kda_out_gate_v3+HEADS=24+K11_RMS_EPS=1e-6f); anything else is
 * K3H_EINVAL. */
K3H_API int k3h_kda_out_gate(k3h_ctx_t ctx, void* stream, const void* attn,
                             const void* gate_partial, const float* gamma_o, void* gated,
                             const int* span_at, int span, float eps);

/* ---- MLA --------------------------------------------------------------------
 * kern_k3_mla_prep_head + kern_k3_mla_prep_gate (k3_mla_prep_v2.cu:91,130;
 * k3_mla_prep_bf16.cu:73,112; manifest op mla_prep, json:404677): partial
 * [B, 5184] f32 (bf16_partial = 0, module k3_mla_prep_v2+...) or bf16
 * (module k3_mla_prep_bf16+...); gammas bf16; slot_mapping i64 [B]; slab bf16
 * paged latent (element offsets layer_off, page_stride; 884736 in the manifest)
 * -> q_norm bf16 [B, 1536], latent rows in the slab, mla_gate bf16 [B, 3072]. */
K3H_API int k3h_mla_prep(k3h_ctx_t ctx, void* stream, int bf16_partial, const void* partial,
                         const void* gamma_q_a, const void* gamma_kv_a,
                         const long long* slot_mapping, void* slab, long long layer_off,
                         long long page_stride, void* q_norm, void* mla_gate, int B);
/* k3h_mla_rope_pack: no reference entry (the reference has no RoPE on this
 * path; its rope columns are a bf16 landing, k3_mla_prep_v2.cu:205-210).
 * latent bf16 [T,512], k_rope bf16 [T,64], q bf16 [T,H,192], gamma_kv bf16
 * [512], positions i64 [T] -> latent_out bf16 [T,576] = RMSNorm(latent) |
 * rope(k_rope), q_out bf16 [T,H,192] = nope | rope(q_rope); interleaved pairs,
 * angle p * theta^(-2j/64). */
K3H_API int k3h_mla_rope_pack(k3h_ctx_t ctx, void* stream, const void* latent,
                              const void* k_rope, const void* q, const void* gamma_kv,
                              const long long* positions, void* latent_out, void* q_out,
                              float theta, float eps, int T, int H);

/* ---- MoE expert GEMMs (MX-scaled matrix cores) ---------------------------------
 * They replace the reference's prebuilt batched GEMMs of manifest ops moe_fc1
 * (k3-tp4-prefill-16k.json:405185; MxE4m3 x MxE2m1 -> MxE4m3 with the siTuGlu
 * activation, kernels.toml:6-9) and moe_fc2 (json:405419; -> bf16), whose
 * per-expert alpha / beta buffers the manifest fills with 4.0 and 25.0
 * (load.fill_f32 calls), and the load-time layouts kern_k3_moe_w_shuffle /
 * kern_k3_moe_sf_shuffle (k3_moe_prefill_v4.cu:69-80, 304-327).
 *
 * k3h_moe_w_tile: row-major e2m1 weights src [experts, n, k/2] (low nibble =
 * even k) -> the MFMA-operand tiled layout dst (same size); gated: src rows are
 * [up; gate] halves (n/2 each) and the tiles alternate up / gate.  n % 32 == 0
 * (n % 64 gated), k % 64 == 0.
 * k3h_moe_sf_tile: E8M0 scales src [experts, n, k/32] -> tiled dst (same size,
 * 8-byte aligned).  n % 128 == 0, k % 128 == 0.
 * k3h_moe_gemm_mx: C[r, :] = a(src(r), :) . w_e^T over the route tiles t <
 * *num_tiles (rows [128 t, 128 t + 128), expert e = cta_batch[t]); a e4m3
 * [rows, K] (16-byte aligned rows) with E8M0 a_sf [rows, K/32]; src(r) =
 * a_rows[r] when a_rows (route_map) is given, else r.  Epilogue:
 *   K3H_GEMM_F32      out f32 [tiles*128, N];
 *   K3H_GEMM_BF16     out bf16 [tiles*128, N] (fc2; 16-byte aligned);
 *   K3H_GEMM_SITU_MX  gated weights: x = bf16(situ(bf16(gate), bf16(up);
 *                     alpha[e], beta[e])) -> out e4m3 [.., N/2] (16-byte
 *                     aligned), out_sf E8M0 [.., N/64] (2-byte aligned),
 *                     quantised as kern_k3_moe_quant (fc1);
 *   K3H_GEMM_F32_SITU_TILING  out f32 [tiles*128, N] (16-byte aligned) from the
 *                     K3H_GEMM_SITU_MX kernel's own tiling, item split and
 *                     operand roles (the same values as K3H_GEMM_F32): checks
 *                     of the fc1 kernel's accumulators; not a serving path.
 * Work items are (tile < min(*num_tiles, max_tiles), 256-column block); the
 * workgroups hand them out per XCD (each XCD a contiguous share of the tiles and
 * columns, so that its L2 holds the operands its workgroups share); the grid
 * (N/256, rows) has enough rows for every XCD's share.  N % 256 == 0,
 * K % 128 == 0, K <= 7168; rows of padding tiles route token 0 and are
 * computed.  a_rows values (when given) must index rows of a / a_sf.  Row
 * offsets into a are 32-bit: without a_rows, max_tiles * 128 * K must not
 * exceed 2^32 - 1 (else K3H_EINVAL); with a_rows, the caller keeps
 * token_count * K below 2^32 (the values are on the device, not checked). */
#define K3H_GEMM_F32 0
#define K3H_GEMM_BF16 1
#define K3H_GEMM_SITU_MX 2
#define K3H_GEMM_F32_SITU_TILING 3
K3H_API int k3h_moe_w_tile(k3h_ctx_t ctx, void* stream, const void* src, void* dst, int experts,
                           int n, int k, int gated);
K3H_API int k3h_moe_sf_tile(k3h_ctx_t ctx, void* stream, const void* src, void* dst, int experts,
                            int n, int k, int gated);
K3H_API int k3h_moe_gemm_mx(k3h_ctx_t ctx, void* stream, int epilogue, const void* a,
                            const void* a_sf, const int* a_rows, const void* wt, const void* wsf,
                            const int* num_tiles, const int* cta_batch, int max_tiles, int E,
                            int N, int K, void* out, void* out_sf, const float* alpha,
                            const float* beta);
/* moe_fc1 / moe_fc2 in the manifest ops' parameter order (json:405185 /
 * 405419), with this build's tiled weights; total_padded and cta_limit are
 * accepted for the signature's sake (the tile count bounds the work). */
K3H_API int k3h_moe_fc1(k3h_ctx_t ctx, void* stream, const void* w13t, const void* w13_sft,
                        const void* a_q, const void* a_sf, void* fc1_out, void* fc1_sf,
                        const int* route_map, const float* alpha, const float* beta,
                        const int* num_non_exiting, const int* total_padded, const int* cta_batch,
                        const int* cta_limit, int max_tiles, int E, int K, int inter);
K3H_API int k3h_moe_fc2(k3h_ctx_t ctx, void* stream, const void* w2t, const void* w2_sft,
                        const void* fc1_out, const void* fc1_sf, void* fc2_out,
                        const int* num_non_exiting, const int* total_padded, const int* cta_batch,
                        const int* cta_limit, int max_tiles, int E, int inter, int cols);

/* k3h_synth_normal: measurement support (host code, no GPU): the synthetic
 * inputs of the benchmark configurations.  n values of mean + std * N(0,1) from
 * the tensor's own xoshiro256** stream (splitmix64-seeded with 24301 ^
 * fnv1a64(name), Box-Muller in double, rounded to f32, then to bf16 when
 * bf16_out); with outlier_p > 0 each element is replaced, with probability
 * outlier_p, by outlier_x * N(0,1) from two more streams (name + "#bernoulli"
 * selects, name + "#outlier" draws).  out: n bf16 (uint16) or f32 values. */
K3H_API int k3h_synth_normal(const char* name, size_t n, float mean, float std_dev, float outlier_p,
                             float outlier_x, int bf16_out, void* out);

/* ---- measurement support --------------------------------------------------
 * k3h_stream_copy: dst[i] = src[i] for n16 16-byte vectors with non-temporal
 * loads and stores, one vector per thread (module k3h_fused).  No reference
 * counterpart: it is the plain copy kernel whose rate is the HBM streaming
 * ceiling the operators are compared with, and whose known byte count
 * calibrates the FETCH_SIZE / WRITE_SIZE counters. */
K3H_API int k3h_stream_copy(k3h_ctx_t ctx, void* stream, const void* src, void* dst,
                            int64_t n16);

#ifdef __cplusplus
}
#endif
#endif
