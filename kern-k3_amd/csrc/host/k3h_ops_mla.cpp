// Typed wrappers: MLA prep (manifest op mla_prep, k3-tp4-prefill-16k.json:404677:
// head launch grid ceil(B/4) x 512 then gate launch grid ceil(B/4) x 384; the
// typed call runs both in the one launch k3h_mla_prep_fused) and the
// latent-norm + RoPE + q packing op (module k3h_mla_rope, grid ceil(T/4) x 256).
#include "k3h_internal.h"

extern "C" {

K3H_API int k3h_mla_prep(k3h_ctx_t ctx, void* stream, int bf16_partial, const void* partial,
                         const void* gamma_q_a, const void* gamma_kv_a,
                         const long long* slot_mapping, void* slab, long long layer_off,
                         long long page_stride, void* q_norm, void* mla_gate, int B) {
  if (!ctx || B < 0 || layer_off < 0 || page_stride < 0 || layer_off % 4 || page_stride % 4)
    return K3H_EINVAL;
  if (B == 0) return K3H_OK;
  if (!k3h_okp(partial, 16) || !k3h_okp(gamma_q_a, 8) || !k3h_okp(gamma_kv_a, 8) ||
      !k3h_okp(slot_mapping, 8) || !k3h_okp(slab, 8) || !k3h_okp(q_norm, 8) ||
      !k3h_okp(mla_gate, 16))
    return K3H_EINVAL;
  const char* key = bf16_partial ? "k3_mla_prep_bf16+INNER=3072+MLA_FUSED=5184"
                                 : "k3_mla_prep_v2+INNER=3072+MLA_FUSED=5184";
  // head and gate in one launch (the manifest's two entries stay in the module)
  K3hArgs h;
  h.ptr(partial).ptr(gamma_q_a).ptr(gamma_kv_a).ptr(slot_mapping).ptr(slab).i64(layer_off);
  h.i64(page_stride).ptr(q_norm).ptr(mla_gate).i32(B);
  return k3h_run(ctx, key, "k3h_mla_prep_fused", k3h_cdiv(B, 4), 1, 1, 512, stream, h);
}

K3H_API int k3h_mla_rope_pack(k3h_ctx_t ctx, void* stream, const void* latent,
                              const void* k_rope, const void* q, const void* gamma_kv,
                              const long long* positions, void* latent_out, void* q_out,
                              float theta, float eps, int T, int H) {
  if (!ctx || T < 0 || H < 1 || !(theta > 0.0f) || !(eps > 0.0f)) return K3H_EINVAL;
  if (T == 0) return K3H_OK;
  if (!k3h_okp(latent, 16) || !k3h_okp(k_rope, 16) || !k3h_okp(q, 16) || !k3h_okp(gamma_kv, 16) ||
      !k3h_okp(positions, 8) || !k3h_okp(latent_out, 16) || !k3h_okp(q_out, 16))
    return K3H_EINVAL;
  K3hArgs a;
  a.ptr(latent).ptr(k_rope).ptr(q).ptr(gamma_kv).ptr(positions).ptr(latent_out).ptr(q_out);
  a.f32(theta).f32(eps).i32(T).i32(H);
  return k3h_run(ctx, "k3h_mla_rope", "k3h_mla_rope_pack", k3h_cdiv(T, 4), 1, 1, 256, stream, a);
}

}  // extern "C"
