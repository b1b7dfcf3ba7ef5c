// Typed wrappers: KDA span gather (K9) and output gate (K11), HEADS = 24
// modules.  The manifest grids (k3-tp4-prefill-16k.json) are span_gather_v2
// 406197 (6, 4, ceil(tokens/16)) x 128 and kda_out_gate_v2 406169 (tokens, 3, 1)
// x 128; the out gate launches the manifest's, the span gather a compact grid of
// 256-thread workgroups that its entry also accepts.
#include "k3h_internal.h"

namespace {
constexpr int kHeads = 24;
constexpr int kInner = kHeads * 128;
constexpr uint32_t kSpanShare = 2;  // 16-row tiles per span-gather workgroup
}  // namespace

extern "C" {

K3H_API int k3h_span_gather(k3h_ctx_t ctx, void* stream, const void* partial, const float* cw,
                            void* kda_base, const int* line_index, long long line_bytes,
                            const float* wsm_partial, void* span_q, void* span_k, void* span_v,
                            void* span_beta, void* span_flow, const int* span_at, int span) {
  if (!ctx || span < 0 || line_bytes < 0 || line_bytes % 16) return K3H_EINVAL;
  if (span == 0) return K3H_OK;
  if (!k3h_okp(partial, 16) || !k3h_okp(cw, 16) || !k3h_okp(kda_base, 16) ||
      !k3h_okp(line_index, 4) || !k3h_okp(wsm_partial, 16) || !k3h_okp(span_q, 16) ||
      !k3h_okp(span_k, 16) || !k3h_okp(span_v, 16) || !k3h_okp(span_beta, 2) ||
      !k3h_okp(span_flow, 16) || !k3h_okp(span_at, 4))
    return K3H_EINVAL;
  K3hArgs a;
  a.ptr(partial).ptr(cw).ptr(kda_base).ptr(line_index).i64(line_bytes).ptr(wsm_partial);
  a.ptr(span_q).ptr(span_k).ptr(span_v).ptr(span_beta).ptr(span_flow).ptr(span_at).i32(span);
  // Two 16-row tiles of a column per 256-thread workgroup (the second tile's
  // taps pass through LDS): one work item per (tile pair, stream, column tile)
  // and one beta / flow item per tile pair, as a 1-D grid.  The entry also runs
  // the manifest's (INNER / 512, 4, ceil(span / 16)) x 128 geometry.
  const uint32_t pairs = k3h_cdiv(k3h_cdiv(span, 16), kSpanShare);
  return k3h_run(ctx, "k3_span_gather_v3+HEADS=24", "kern_k3_span_gather",
                 (3 * (kInner / 512) + 1) * pairs, 1, 1, 128 * kSpanShare, stream, a);
}

K3H_API int k3h_kda_out_gate(k3h_ctx_t ctx, void* stream, const void* attn,
                             const void* gate_partial, const float* gamma_o, void* gated,
                             const int* span_at, int span, float eps) {
  // eps selects the module: the norm's eps is compiled in (k3_kda_out_gate_v3.cu:25).
  const char* key;
  if (eps == 1e-5f) key = "k3_kda_out_gate_v3+HEADS=24";
  else if (eps == 1e-6f) key = "k3_kda_out_gate_v3+HEADS=24+K11_RMS_EPS=1e-6f";
  else return K3H_EINVAL;
  if (!ctx || span < 0) return K3H_EINVAL;
  if (span == 0) return K3H_OK;
  if (!k3h_okp(attn, 16) || !k3h_okp(gate_partial, 16) || !k3h_okp(gamma_o, 16) ||
      !k3h_okp(gated, 16) || !k3h_okp(span_at, 4))
    return K3H_EINVAL;
  K3hArgs a;
  a.ptr(attn).ptr(gate_partial).ptr(gamma_o).ptr(gated).ptr(span_at).i32(span);
  return k3h_run(ctx, key, "kern_k3_kda_out_gate", (uint32_t)span,
                 kHeads / 8, 1, 128, stream, a);
}

}  // extern "C"
