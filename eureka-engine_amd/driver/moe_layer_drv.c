/* moe_layer_drv.c -- a standalone C host for one MoE layer, in the role of llb_moe_run
 * (host/llb_host.c:622-724), over the C ABI only: the backend contract of host/llb_backend.h through
 * include/llb_backend_hip.h (LLB_LAUNCH, llb_alloc_zero, llb_read, llb_sync) and the layer entry points
 * of include/llb_moe_hip.h.
 *
 * It lays out one layer's Bytes region the way a table row points into it: the shared expert's gate,
 * up and down matrices (words 3..5), the router rows (word 21) and the shared gate row (word 22). It
 * fills that region, the expert stacks and the inputs with the library's seeded generator (the same
 * streams as the Python test harness: stream = layer * 16 + tensor slot). It writes the 32 table
 * words (tools/gguf2pack.c:1142-1146). The generator writes the token rows into staging buffers; a
 * kernel of drv_kernels.hsaco (next to this binary), looked up by name and launched with LLB_LAUNCH's
 * argument-address convention (a by-value struct, a float), stages them into the layer's inputs. Then
 * it runs the layer through llb_moe_run_table, which does the
 * admission check, the field decode and the forward. Then it writes y [T][dm], ids [T][nk] and
 * wt [T][nk] to a file and prints a one-line summary.
 *
 * usage: moe_layer_drv <c2|c5> <seed> <T> <tier: 0 exact, 1 q8, 2 f16> <out.bin>
 * Exit status 0 on success, 1 on a library error (named on stderr), 2 on bad arguments.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "../../include/llb_backend_hip.h"

enum { ST_ROUTER, ST_SHGATE, ST_G, ST_U, ST_D, ST_SG, ST_SU, ST_SD, ST_H2, ST_X1 };
#define W_SIGMA 0.02f

static uint64_t row_bytes(uint32_t fm, uint32_t cols) {
  switch (fm) {
    case LLB_FM_F32: return (uint64_t)cols * 4;
    case LLB_FM_Q8_0: return (uint64_t)cols / 32 * 34;
    case LLB_FM_Q4_K: return (uint64_t)cols / 256 * 144;
    case LLB_FM_Q5_K: return (uint64_t)cols / 256 * 176;
    case LLB_FM_Q6_K: return (uint64_t)cols / 256 * 210;
    default: return 0;
  }
}
static uint64_t al256(uint64_t n) { return (n + 255) & ~(uint64_t)255; }

static int ok(int rc, const char* what) {
  if (rc != 0) {
    fprintf(stderr, "moe_layer_drv: %s failed (%d): %s\n", what, rc, llb_hip_last_error());
    exit(1);
  }
  return rc;
}
static llb_dptr alloc(uint64_t n) {
  llb_dptr p = llb_alloc_zero((size_t)n);
  if (!p) {
    fprintf(stderr, "moe_layer_drv: alloc of %llu bytes failed: %s\n", (unsigned long long)n, llb_hip_last_error());
    exit(1);
  }
  return p;
}

int main(int argc, char** argv) {
  if (argc != 6) {
    fprintf(stderr, "usage: %s <c2|c5> <seed> <T> <tier: 0 exact, 1 q8, 2 f16> <out.bin>\n", argv[0]);
    return 2;
  }
  /* the benchmark shapes with a shared expert (the admission needs one): config 2 and config 5 */
  uint32_t dm = 2048, ne, nk, ef = 512, sf = 512;
  const uint32_t fg = LLB_FM_Q4_K, fu = LLB_FM_Q4_K, fd = LLB_FM_Q6_K;
  const uint32_t fsg = LLB_FM_Q4_K, fsu = LLB_FM_Q4_K, fsd = LLB_FM_Q6_K;
  if (!strcmp(argv[1], "c2")) {
    ne = 256;
    nk = 8;
  } else if (!strcmp(argv[1], "c5")) {
    ne = 512;
    nk = 10;
  } else {
    fprintf(stderr, "moe_layer_drv: unknown shape %s\n", argv[1]);
    return 2;
  }
  const uint64_t seed = strtoull(argv[2], NULL, 10);
  const long T = strtol(argv[3], NULL, 10);
  const int tier = atoi(argv[4]);
  if (T < 1 || T > 65536 || tier < 0 || tier > 2) {
    fprintf(stderr, "moe_layer_drv: T in 1..65536, tier 0..2\n");
    return 2;
  }
  ok(llb_hip_init(0), "llb_hip_init");

  /* the layer's Bytes: shared gate / up / down, router rows, shared gate row */
  const uint64_t o_sg = 0;
  const uint64_t o_su = o_sg + al256(sf * row_bytes(fsg, dm));
  const uint64_t o_sd = o_su + al256(sf * row_bytes(fsu, dm));
  const uint64_t o_r = o_sd + al256(dm * row_bytes(fsd, sf));
  const uint64_t o_g = o_r + al256((uint64_t)ne * dm * 4);
  const uint64_t len = o_g + (uint64_t)dm * 4;
  const llb_dptr base = alloc(len);
  const llb_dptr G = alloc((uint64_t)ne * ef * row_bytes(fg, dm));
  const llb_dptr U = alloc((uint64_t)ne * ef * row_bytes(fu, dm));
  const llb_dptr D = alloc((uint64_t)ne * dm * row_bytes(fd, ef));
  ok(llb_moe_hip_gen_rows(LLB_FM_F32, seed, ST_ROUTER, 0, ne, dm, W_SIGMA, base + o_r), "router rows");
  ok(llb_moe_hip_gen_rows(LLB_FM_F32, seed, ST_SHGATE, 0, 1, dm, W_SIGMA, base + o_g), "shared gate row");
  ok(llb_moe_hip_gen_rows(fg, seed, ST_G, 0, (uint64_t)ne * ef, dm, W_SIGMA, G), "gate stack");
  ok(llb_moe_hip_gen_rows(fu, seed, ST_U, 0, (uint64_t)ne * ef, dm, W_SIGMA, U), "up stack");
  ok(llb_moe_hip_gen_rows(fd, seed, ST_D, 0, (uint64_t)ne * dm, ef, W_SIGMA, D), "down stack");
  ok(llb_moe_hip_gen_rows(fsg, seed, ST_SG, 0, sf, dm, W_SIGMA, base + o_sg), "shared gate");
  ok(llb_moe_hip_gen_rows(fsu, seed, ST_SU, 0, sf, dm, W_SIGMA, base + o_su), "shared up");
  ok(llb_moe_hip_gen_rows(fsd, seed, ST_SD, 0, dm, sf, W_SIGMA, base + o_sd), "shared down");

  /* the table row: offsets into Bytes with the format in the top four bits */
  uint32_t w[32];
  memset(w, 0, sizeof w);
  w[3] = (uint32_t)o_sg | fsg << 28;
  w[4] = (uint32_t)o_su | fsu << 28;
  w[5] = (uint32_t)o_sd | fsd << 28;
  w[21] = (uint32_t)o_r | (uint32_t)LLB_FM_F32 << 28;
  w[22] = (uint32_t)o_g | (uint32_t)LLB_FM_F32 << 28;
  w[26] = fg | fu << 4 | fd << 8 | 1u << 13;
  w[27] = ne;
  w[28] = ef;
  w[29] = sf;
  w[30] = nk;
  const uint32_t df = 4 * dm; /* the dense FFN width cap the admission compares ef and sf with */
  if (llb_moe_table_check(w, dm, df, len) != 0) {
    fprintf(stderr, "moe_layer_drv: the table row fails the admission check\n");
    return 1;
  }

  const uint64_t n = (uint64_t)T * dm;
  const llb_dptr h2 = alloc(n * 4), x1 = alloc(n * 4), y = alloc(n * 4);
  const llb_dptr ids = alloc((uint64_t)T * nk * 4), wt = alloc((uint64_t)T * nk * 4);
  const llb_dptr hs = alloc(n * 4), xs = alloc(n * 4);
  ok(llb_moe_hip_gen_gauss(seed, ST_H2, 0, n, 1.0f, hs), "h2");
  ok(llb_moe_hip_gen_gauss(seed, ST_X1, 0, n, 1.0f, xs), "x1");
  /* the staging kernel, by name from the code object beside this binary */
  char path[4096];
  const ssize_t pl = readlink("/proc/self/exe", path, sizeof path - 32);
  if (pl <= 0) return 1;
  path[pl] = 0;
  char* slash = strrchr(path, '/');
  strcpy(slash ? slash + 1 : path, "drv_kernels.hsaco");
  uint64_t mod = 0;
  void* k_stage = NULL;
  ok(llb_hip_module_load(path, &mod), "llb_hip_module_load");
  ok(llb_hip_module_function(mod, "llb_drv_stage", &k_stage), "llb_hip_module_function");
  struct {
    llb_dptr src, dst;
    uint32_t n, pad;
  } sa = {hs, h2, (uint32_t)n, 0}, sb2 = {xs, x1, (uint32_t)n, 0};
  float one = 1.0f;
  if (!LLB_LAUNCH(k_stage, (n + 255) / 256, 2, 256, &sa, &sb2, &one)) {
    fprintf(stderr, "moe_layer_drv: LLB_LAUNCH failed: %s\n", llb_hip_last_error());
    return 1;
  }
  llb_moe_layer L;
  ok(llb_moe_layer_from_table(w, dm, base, G, U, D, &L), "llb_moe_layer_from_table");
  const size_t sb = llb_moe_hip_scratch_bytes(&L, (uint32_t)T, tier);
  const llb_dptr scratch = alloc(sb);
  ok(llb_moe_run_table(w, dm, df, len, base, G, U, D, (uint32_t)T, h2, x1, y, ids, wt, scratch, sb, tier),
     "llb_moe_run_table");
  if (!llb_sync()) {
    fprintf(stderr, "moe_layer_drv: llb_sync failed: %s\n", llb_hip_last_error());
    return 1;
  }

  float* hy = (float*)malloc(n * 4);
  uint32_t* hid = (uint32_t*)malloc((size_t)T * nk * 4);
  float* hwt = (float*)malloc((size_t)T * nk * 4);
  if (!hy || !hid || !hwt) return 1;
  if (!llb_read(hy, y, n * 4) || !llb_read(hid, ids, (size_t)T * nk * 4) || !llb_read(hwt, wt, (size_t)T * nk * 4)) {
    fprintf(stderr, "moe_layer_drv: llb_read failed: %s\n", llb_hip_last_error());
    return 1;
  }
  FILE* f = fopen(argv[5], "wb");
  if (!f || fwrite(hy, 4, n, f) != n || fwrite(hid, 4, (size_t)T * nk, f) != (size_t)T * nk ||
      fwrite(hwt, 4, (size_t)T * nk, f) != (size_t)T * nk || fclose(f) != 0) {
    fprintf(stderr, "moe_layer_drv: cannot write %s\n", argv[5]);
    return 1;
  }
  double s = 0.0;
  for (uint64_t i = 0; i < n; i++) s += hy[i];
  printf("moe_layer_drv %s seed %llu T %ld tier %d: ids[0] = %u, wt[0] = %.6g, sum y = %.6f\n", argv[1],
         (unsigned long long)seed, T, tier, hid[0], hwt[0], s);
  free(hy);
  free(hid);
  free(hwt);
  return 0;
}
