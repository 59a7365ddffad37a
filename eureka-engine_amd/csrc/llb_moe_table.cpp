// llb_moe_table.cpp -- the layer's table row as the reference host reads it (host code, no GPU).
//
// table.bin holds 32 u32 words a layer (tools/gguf2pack.c:1142-1146, :1294-1312); the engine keeps
// pt[f] = word f + 1 (tools/payload-moeany.patch:65-71) and llb_moe_run reads its fields from pt
// (host/llb_host.c:623-627). These functions take the raw 32 words of one layer:
//   w[3], w[4], w[5]  shared gate / up / down: offset | fm << 28 (Offs words 2..4)
//   w[21] router offset | fm << 28 (F32), w[22] the shared expert's gate row
//   w[26] gate | up << 4 | down << 8, bit 12 fused gate+up, bit 13 set
//   w[27] expert count, w[28] expert ff, w[29] shared ff, w[30] experts used
#include "../../include/llb_moe_hip.h"

static bool moe_fm_ok(uint32_t f) {
  return f == LLB_FM_Q8_0 || f == LLB_FM_Q4_K || f == LLB_FM_Q5_K || f == LLB_FM_Q6_K;
}

extern "C" {

// pass_mail's admission of a routed-expert layer (tools/payload-moeany.patch:26-50): 0, or 8 (the
// engine's Mail.bad code, named at host/llb_host.c:3285-3287). df: the dense FFN width cap; len: the
// layer's byte length (the router and shared gate rows must lie inside it)
int llb_moe_table_check(const uint32_t* w, uint32_t dm, uint32_t df, uint64_t len) {
  if (!w) return 8;
  const uint32_t ne = w[27], nk = w[30], ef = w[28], sf = w[29], fx = w[26];
  if (ne == 0) return 0;  // not a routed-expert layer
  const uint32_t fg = fx & 15, fu = fx >> 4 & 15, fd = fx >> 8 & 15, fz = fx >> 12 & 1;
  const uint32_t ro = w[21] & 0x0fffffffu, go = w[22] & 0x0fffffffu;
  const bool ok = ne >= 1 && nk >= 1 && nk <= ne && ef >= 256 && ef % 256 == 0 && ef <= df && sf >= 256 &&
                  sf % 256 == 0 && sf <= df && (fx >> 13 & 1) && moe_fm_ok(fg) && moe_fm_ok(fu) && moe_fm_ok(fd) &&
                  (!fz || fu == fg) && w[21] >> 28 == LLB_FM_F32 && w[22] >> 28 == LLB_FM_F32 && ro % 4 == 0 &&
                  go % 4 == 0 && (uint64_t)ro + (uint64_t)ne * dm * 4 <= len && (uint64_t)go + (uint64_t)dm * 4 <= len;
  return ok ? 0 : 8;
}

// llb_moe_run's decode of the row (host/llb_host.c:623-627): the layer's Bytes start at base; the
// stacks come from llb_moe_load (host/llb_host.c:491-586) as device addresses (U ignored when fused)
int llb_moe_layer_from_table(const uint32_t* w, uint32_t dm, llb_dptr base, llb_dptr G, llb_dptr U, llb_dptr D,
                             llb_moe_layer* out) {
  if (!w || !out) return LLB_HIP_EINVAL;
  const uint32_t m = 0x0fffffffu;
  llb_moe_layer L = {};
  L.dm = dm;
  L.ne = w[27];
  L.ef = w[28];
  L.sf = w[29];
  L.nk = w[30];
  L.fx = w[26];
  L.fsg = w[3] >> 28;
  L.fsu = w[4] >> 28;
  L.fsd = w[5] >> 28;
  L.router = base + (w[21] & m);
  L.shgate = L.sf ? base + (w[22] & m) : 0;
  L.G = G;
  L.U = (w[26] >> 12 & 1) ? 0 : U;
  L.D = D;
  L.SG = L.sf ? base + (w[3] & m) : 0;
  L.SU = L.sf ? base + (w[4] & m) : 0;
  L.SD = L.sf ? base + (w[5] & m) : 0;
  *out = L;
  return 0;
}

// one layer from its table row: the check, the decode, llb_moe_hip_forward
int llb_moe_run_table(const uint32_t* w, uint32_t dm, uint32_t df, uint64_t len, llb_dptr base, llb_dptr G, llb_dptr U,
                      llb_dptr D, uint32_t T, llb_dptr h2, llb_dptr x1, llb_dptr y, llb_dptr ids, llb_dptr wt,
                      llb_dptr scratch, size_t scratch_bytes, int tier) {
  if (llb_moe_table_check(w, dm, df, len) != 0) return LLB_HIP_EINVAL;
  llb_moe_layer L;
  int rc = llb_moe_layer_from_table(w, dm, base, G, U, D, &L);
  if (rc) return rc;
  return llb_moe_hip_forward(&L, T, h2, x1, y, ids, wt, scratch, scratch_bytes, tier);
}

}  // extern "C"
