// llb_moe_gguf.cpp -- GGUF expert stacks into the layer (llb_moe_load / moe_fill,
// host/llb_host.c:446-586; llb_gg_tensor, host/llb_gguf.c:854-865). Host code.
//
// The file is read with pread: the header (metadata and tensor table) is parsed with every length and
// count checked against the file size, then tensors are found by name. A layer's stacks are
// blk.N.ffn_gate_exps / ffn_up_exps / ffn_down_exps (or ffn_gate_up_exps for the fused stack), checked
// against the layer's declared formats and byte counts as the reference does, and placed:
//   device  hipMalloc + pread in 64 MiB pieces + upload (the reference's mode 0);
//   host    pinned, device-mapped host memory (hipHostMalloc mapped | portable), pread in place (mode 1);
//   stream  the file mapped read-only; per decoded token the k chosen experts are copied into device
//           staging slots and the experts run on slot ids 0..k-1 (mode 2; llb_moe_hip_forward does it).
// The router (ffn_gate_inp), the shared gate row (ffn_gate_inp_shexp) and the shared expert
// (ffn_{gate,up,down}_shexp) are loaded the same way when the file holds them and the layer does not
// already point at them (the reference takes those from its pack; a GGUF-only caller takes them here).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "../../include/llb_moe_hip.h"
#include "moe_kernels.h"

uint64_t llb_row_bytes(uint32_t fm, uint32_t cols);
#define row_bytes llb_row_bytes

struct GgTensor {
  std::string name;
  uint32_t type, nd;
  uint64_t dims[4];
  uint64_t off;    // from the file start
  uint64_t bytes;
};
struct llb_gguf {
  int fd;
  uint64_t size;
  uint32_t version, alignment;
  std::vector<GgTensor> t;
  std::string arch;                                   // general.architecture
  std::vector<std::pair<std::string, int64_t>> ints;  // scalar integer metadata, by key
};
static bool gg_int(const llb_gguf* g, const std::string& key, int64_t* v) {
  for (const auto& kv : g->ints)
    if (kv.first == key) return (*v = kv.second, true);
  return false;
}

// ggml type -> (block bytes, block elements); 0 for types this path does not read
static bool gg_block(uint32_t ty, uint64_t& bb, uint64_t& be) {
  switch (ty) {
    case 0: bb = 4; be = 1; return true;      // F32
    case 1: bb = 2; be = 1; return true;      // F16
    case 8: bb = 34; be = 32; return true;    // Q8_0
    case 12: bb = 144; be = 256; return true; // Q4_K
    case 13: bb = 176; be = 256; return true; // Q5_K
    case 14: bb = 210; be = 256; return true; // Q6_K
    case 11: bb = 110; be = 256; return true; // Q3_K
    case 23: bb = 136; be = 256; return true; // IQ4_XS
    case 42: bb = 18; be = 64; return true;   // Q2_0
    case 142: bb = 34; be = 128; return true; // PQ2_0
    case 30: bb = 2; be = 1; return true;     // BF16
    default: return false;
  }
}
// ggml type -> LLB_FM_* (host/llb_formats.h:5-14); -1 when the path has no decoder for it
static int gg_fm(uint32_t ty) {
  switch (ty) {
    case 0: return LLB_FM_F32;
    case 8: return LLB_FM_Q8_0;
    case 12: return LLB_FM_Q4_K;
    case 13: return LLB_FM_Q5_K;
    case 14: return LLB_FM_Q6_K;
    default: return -1;
  }
}

struct Rd {
  int fd;
  uint64_t size, pos;
  bool bad;
  bool get(void* p, uint64_t n) {
    if (bad || n > size || pos > size - n) return (bad = true, false);
    uint8_t* q = (uint8_t*)p;
    for (uint64_t k = 0; k < n;) {
      const ssize_t r = pread(fd, q + k, (size_t)(n - k), (off_t)(pos + k));
      if (r <= 0) return (bad = true, false);
      k += (uint64_t)r;
    }
    pos += n;
    return true;
  }
  template <class T> T v() {
    T x{};
    get(&x, sizeof x);
    return x;
  }
  bool str(std::string* s) {
    const uint64_t n = v<uint64_t>();
    if (bad || n > (1u << 20) || n > size - pos) return (bad = true, false);
    if (!s) return (pos += n, true);
    s->resize((size_t)n);
    return get(&(*s)[0], n);
  }
  // skips a metadata value of type ty (arrays nest at most 4 deep)
  bool skip(uint32_t ty, int depth = 0) {
    static const uint8_t sz[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    if (ty == 8) return str(nullptr);
    if (ty == 9) {
      const uint32_t et = v<uint32_t>();
      const uint64_t n = v<uint64_t>();
      if (bad || depth >= 4 || et > 12) return (bad = true, false);
      if (et != 8 && et != 9) {
        if (n > (size - pos) / sz[et]) return (bad = true, false);
        pos += n * sz[et];
        return true;
      }
      for (uint64_t i = 0; i < n && !bad; i++) skip(et, depth + 1);
      return !bad;
    }
    if (ty > 12) return (bad = true, false);
    if (sz[ty] > size - pos) return (bad = true, false);
    pos += sz[ty];
    return true;
  }
};

extern "C" {

llb_gguf* llb_gguf_open(const char* path) {
  if (!path) return (llb_fail_msg(LLB_HIP_EINVAL, "gguf: null path"), nullptr);
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return (llb_fail_msg(LLB_HIP_EINVAL, "gguf: cannot open the file"), nullptr);
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    return (llb_fail_msg(LLB_HIP_EINVAL, "gguf: cannot stat the file"), nullptr);
  }
  Rd r{fd, (uint64_t)st.st_size, 0, false};
  const uint32_t magic = r.v<uint32_t>(), version = r.v<uint32_t>();
  const uint64_t nt = r.v<uint64_t>(), nkv = r.v<uint64_t>();
  const char* why = nullptr;
  if (r.bad || magic != 0x46554747u) why = "gguf: not a GGUF file";
  else if (version < 2 || version > 3) why = "gguf: only versions 2 and 3";
  else if (nt > (1u << 24) || nkv > (1u << 24)) why = "gguf: implausible tensor or key count";
  uint32_t alignment = 32;
  std::string arch;
  std::vector<std::pair<std::string, int64_t>> ints;
  for (uint64_t i = 0; !why && i < nkv; i++) {
    std::string key;
    r.str(&key);
    const uint32_t ty = r.v<uint32_t>();
    if (key == "general.alignment" && ty == 4) {
      alignment = r.v<uint32_t>();
      if (alignment == 0 || (alignment & (alignment - 1))) why = "gguf: general.alignment not a power of two";
    } else if (key == "general.architecture" && ty == 8) {
      r.str(&arch);
    } else if (ty <= 5 || ty == 10 || ty == 11) {  // scalar integers, kept by key
      int64_t v = 0;
      switch (ty) {
        case 0: v = r.v<uint8_t>(); break;
        case 1: v = r.v<int8_t>(); break;
        case 2: v = r.v<uint16_t>(); break;
        case 3: v = r.v<int16_t>(); break;
        case 4: v = r.v<uint32_t>(); break;
        case 5: v = r.v<int32_t>(); break;
        case 10: v = (int64_t)r.v<uint64_t>(); break;
        default: v = r.v<int64_t>(); break;
      }
      ints.emplace_back(key, v);
    } else {
      r.skip(ty);
    }
    if (r.bad) why = "gguf: truncated or malformed metadata";
  }
  auto* g = new llb_gguf{fd, (uint64_t)st.st_size, version, alignment, {}, arch, ints};
  if (!why) g->t.reserve((size_t)nt);
  for (uint64_t i = 0; !why && i < nt; i++) {
    GgTensor t{};
    r.str(&t.name);
    t.nd = r.v<uint32_t>();
    if (r.bad || t.nd == 0 || t.nd > 4) {
      why = "gguf: malformed tensor table";
      break;
    }
    uint64_t ne = 1;
    for (uint32_t d = 0; d < t.nd; d++) {
      t.dims[d] = r.v<uint64_t>();
      if (t.dims[d] == 0 || t.dims[d] > (1ull << 40) || ne > (1ull << 48) / t.dims[d]) why = "gguf: implausible tensor shape";
      else ne *= t.dims[d];
    }
    t.type = r.v<uint32_t>();
    t.off = r.v<uint64_t>();
    if (r.bad) why = "gguf: truncated tensor table";
    uint64_t bb = 0, be = 1;
    if (!why && gg_block(t.type, bb, be)) {
      if (t.dims[0] % be) why = "gguf: a row is not whole blocks";
      else t.bytes = ne / be * bb;
    }
    g->t.push_back(t);
  }
  if (!why) {
    const uint64_t data = (r.pos + alignment - 1) / alignment * alignment;
    for (auto& t : g->t) {
      if (t.off % alignment || t.off > g->size || data > g->size - t.off) {
        why = "gguf: a tensor offset outside the file";
        break;
      }
      t.off += data;
      if (t.bytes > g->size - t.off) {
        why = "gguf: a tensor runs past the end of the file";
        break;
      }
    }
  }
  if (why) {
    close(fd);
    delete g;
    return (llb_fail_msg(LLB_HIP_EINVAL, why), nullptr);
  }
  return g;
}

void llb_gguf_close(llb_gguf* g) {
  if (!g) return;
  close(g->fd);
  delete g;
}

uint64_t llb_gguf_count(const llb_gguf* g) { return g ? g->t.size() : 0; }

int llb_gguf_tensor_at(const llb_gguf* g, uint64_t i, char* name, size_t cap, uint64_t* offset, uint64_t* bytes,
                       uint32_t* type, uint32_t* nd, uint64_t* dims) {
  if (!g || i >= g->t.size()) return llb_fail_msg(LLB_HIP_EINVAL, "gguf: no such tensor index");
  const GgTensor& t = g->t[i];
  if (name && cap) snprintf(name, cap, "%s", t.name.c_str());
  if (offset) *offset = t.off;
  if (bytes) *bytes = t.bytes;
  if (type) *type = t.type;
  if (nd) *nd = t.nd;
  if (dims)
    for (uint32_t d = 0; d < 4; d++) dims[d] = d < t.nd ? t.dims[d] : 1;
  return 0;
}

// table.bin rows from the GGUF header (the reference's sidecar writer, tools/gguf2pack.c:1134-1346 for
// qwen35moe): the virtual pack layout is the non-layer tensors, then each layer's trunk (every tensor but
// the *_exps stacks), file order within each, then every *_exps stack in layer order, each at a 64-byte
// boundary. A row's word 0 is its layer's trunk bytes; words 1..20 the dense tensors' offsets in the trunk
// (| format << 28), the shared expert under the dense ffn names (words 3..5); 21 the router, 22 the shared
// gate row; 26 the expert formats (gate | up << 4 | down << 8, bit 12 fused gate+up, bit 13); 27 experts,
// 28 expert ff, 29 shared ff, 30 experts used. The nextn (MTP) blocks at the end are left out.
// The ggml types the table places and their LLB_FM_* codes (host/llb_formats.h:5-14): the reference's
// writer knows these and BF16 (tools/gguf2pack.c:377-379), but BF16 has no registry entry and its writer
// does not finish on a file that holds one (its manifest reads the missing entry's code,
// tools/gguf2pack.c:843,861), so BF16 is refused here.
static int gg_fm_any(uint32_t ty) {
  switch (ty) {
    case 0: return 0;    // F32
    case 1: return 2;    // F16
    case 8: return 1;    // Q8_0
    case 12: return 3;   // Q4_K
    case 13: return 9;   // Q5_K
    case 14: return 4;   // Q6_K
    case 11: return 5;   // Q3_K
    case 42: return 6;   // Q2_0
    case 142: return 7;  // PQ2_0
    case 23: return 8;   // IQ4_XS
    default: return -1;
  }
}
static int gg_layer(const std::string& n) {
  if (n.compare(0, 4, "blk.") != 0) return -1;
  int L = 0;
  size_t i = 4;
  if (i >= n.size() || n[i] < '0' || n[i] > '9') return -1;
  while (i < n.size() && n[i] >= '0' && n[i] <= '9' && L < (1 << 20)) L = 10 * L + (n[i++] - '0');
  return i < n.size() && n[i] == '.' ? L : -1;
}
static bool gg_exps(const std::string& n) { return n.size() > 12 && n.compare(n.size() - 12, 12, "_exps.weight") == 0; }

int llb_moe_table_from_gguf(const llb_gguf* g, uint32_t* table, uint32_t cap, uint32_t* nlayers) {
  static const char* offs[20] = {
      "attn_norm.weight", "post_attention_norm.weight", "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight",
      "attn_qkv.weight", "attn_gate.weight", "ssm_beta.weight", "ssm_alpha.weight", "ssm_a", "ssm_dt.bias",
      "ssm_conv1d.weight", "ssm_norm.weight", "ssm_out.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight",
      "attn_q_norm.weight", "attn_k_norm.weight", "attn_output.weight"};
  static const char* shn[3] = {"ffn_gate_shexp.weight", "ffn_up_shexp.weight", "ffn_down_shexp.weight"};
  if (!g || !nlayers) return llb_fail_msg(LLB_HIP_EINVAL, "table: null file or count");
  if (g->arch != "qwen35moe") return llb_fail_msg(LLB_HIP_EINVAL, "table: general.architecture is not qwen35moe");
  int64_t L0 = 0, ne = 0, nk = 0, ef = 0, sf = 0, mtp = 0;
  const std::string a = g->arch + ".";
  int64_t D = 0;
  if (!gg_int(g, a + "block_count", &L0) || !gg_int(g, a + "embedding_length", &D) || !gg_int(g, a + "expert_count", &ne) ||
      !gg_int(g, a + "expert_used_count", &nk) || !gg_int(g, a + "expert_feed_forward_length", &ef) ||
      !gg_int(g, a + "expert_shared_feed_forward_length", &sf))
    return llb_fail_msg(LLB_HIP_EINVAL, "table: a qwen35moe expert / block count key is missing");
  gg_int(g, a + "nextn_predict_layers", &mtp);
  if (L0 < 1 || L0 > 4096 || D < 1 || ne < 1 || ne > 0xffffffffll || nk < 1 || nk > ne || ef < 1 || sf < 1 || mtp < 0 ||
      mtp >= L0)
    return llb_fail_msg(LLB_HIP_EINVAL, "table: implausible block / expert counts");
  {  // a name twice is refused (tools/gguf2pack.c:1187-1189)
    std::vector<const std::string*> nm;
    for (const auto& t : g->t) nm.push_back(&t.name);
    std::sort(nm.begin(), nm.end(), [](const std::string* x, const std::string* y) { return *x < *y; });
    for (size_t i = 1; i < nm.size(); i++)
      if (*nm[i] == *nm[i - 1]) return llb_fail_msg(LLB_HIP_EINVAL, ("table: " + *nm[i] + ": duplicate tensor").c_str());
  }
  const uint32_t nl = (uint32_t)(L0 - mtp);
  *nlayers = nl;
  if (!table || cap < nl) return llb_fail_msg(LLB_HIP_EINVAL, "table: the table holds fewer rows than layers");
  // the virtual layout: a stable order by (routed stack, layer), every tensor at a 64-byte boundary
  const size_t n = g->t.size();
  std::vector<size_t> ord(n);
  std::vector<int> lay(n);
  std::vector<char> ex(n);
  for (size_t i = 0; i < n; i++) {
    ord[i] = i;
    lay[i] = gg_layer(g->t[i].name);
    ex[i] = lay[i] >= 0 && gg_exps(g->t[i].name);
    if (!g->t[i].bytes || gg_fm_any(g->t[i].type) < 0)
      return llb_fail_msg(LLB_HIP_EINVAL, ("table: " + g->t[i].name + ": a tensor type the table cannot place").c_str());
  }
  std::stable_sort(ord.begin(), ord.end(), [&](size_t x, size_t y) {
    return ex[x] != ex[y] ? ex[x] < ex[y] : lay[x] < lay[y];
  });
  std::vector<uint64_t> pos(n);
  uint64_t at = 0;
  for (size_t k = 0; k < n; k++) {
    at = (at + 63) / 64 * 64;
    pos[ord[k]] = at;
    at += g->t[ord[k]].bytes;
  }
  std::vector<uint64_t> lo(nl, UINT64_MAX), hi(nl, 0);
  for (size_t i = 0; i < n; i++)
    if (lay[i] >= 0 && (uint32_t)lay[i] < nl && !ex[i]) {
      lo[lay[i]] = std::min(lo[lay[i]], pos[i]);
      hi[lay[i]] = std::max(hi[lay[i]], pos[i] + g->t[i].bytes);
    }
  memset(table, 0, (size_t)nl * 128);
  for (uint32_t L = 0; L < nl; L++) {
    if (lo[L] == UINT64_MAX) return llb_fail_msg(LLB_HIP_EINVAL, "table: a layer without trunk tensors");
    if (hi[L] - lo[L] > (1ull << 31)) return llb_fail_msg(LLB_HIP_EINVAL, "table: a layer's trunk is over 2 GiB");
    table[L * 32] = (uint32_t)(hi[L] - lo[L]);
  }
  std::vector<uint8_t> need((size_t)nl * 6, 0);  // router, shared gate row, gate, up, gate+up, down
  for (size_t i = 0; i < n; i++) {
    if (lay[i] < 0 || (uint32_t)lay[i] >= nl) continue;
    const uint32_t L = (uint32_t)lay[i];
    const std::string& nm = g->t[i].name;
    const std::string s = nm.substr(nm.find('.', 4) + 1);
    uint32_t* w = table + L * 32;
    const uint32_t fm = (uint32_t)gg_fm_any(g->t[i].type);
    int j = 0;
    while (j < 20 && s != offs[j]) j++;
    for (int k = 0; k < 3 && j == 20; k++)
      if (s == shn[k]) j = 2 + k;
    const bool router = s == "ffn_gate_inp.weight", shgate = s == "ffn_gate_inp_shexp.weight";
    if (j < 20 || router || shgate) {
      if (j == 20) j = router ? 20 : 21;
      const uint64_t rel = pos[i] - lo[L];
      if (rel >= (1ull << 28)) return llb_fail_msg(LLB_HIP_EINVAL, "table: an offset in a layer at or past 2^28");
      w[1 + j] = (uint32_t)rel | fm << 28;
      if (router) need[L * 6 + 0] = 1;
      if (shgate) need[L * 6 + 1] = 1;
      // the router is F32 [expert_count x d_model], the shared gate row F32 [d_model] (or [1 x d_model])
      // (tools/gguf2pack.c:1253-1257); GGUF dims run columns first
      const GgTensor& t = g->t[i];
      if (router && (t.type != 0 || t.nd != 2 || t.dims[0] != (uint64_t)D || t.dims[1] != (uint64_t)ne))
        return llb_fail_msg(LLB_HIP_EINVAL, ("table: " + nm + ": the router must be F32 [expert_count x d_model]").c_str());
      if (shgate && (t.type != 0 || t.dims[0] != (uint64_t)D || !(t.nd == 1 || (t.nd == 2 && t.dims[1] == 1))))
        return llb_fail_msg(LLB_HIP_EINVAL, ("table: " + nm + ": the shared-expert gate must be F32 [d_model]").c_str());
      continue;
    }
    const int x = s == "ffn_gate_exps.weight" || s == "ffn_gate_up_exps.weight" ? 0
                  : s == "ffn_up_exps.weight"                                 ? 1
                  : s == "ffn_down_exps.weight"                               ? 2
                                                                              : -1;
    if (x < 0) return llb_fail_msg(LLB_HIP_EINVAL, ("table: " + nm + ": a tensor outside the MoE table").c_str());
    const bool fz = s == "ffn_gate_up_exps.weight";
    need[L * 6 + (fz ? 4 : x == 0 ? 2 : x == 1 ? 3 : 5)] = 1;
    {  // [expert_count x rows x cols] in Q8_0 / Q4_K / Q5_K / Q6_K (tools/gguf2pack.c:1258-1268)
      const GgTensor& t = g->t[i];
      const uint64_t rows = x == 2 ? (uint64_t)D : fz ? 2 * (uint64_t)ef : (uint64_t)ef;
      const uint64_t cols = x == 2 ? (uint64_t)ef : (uint64_t)D;
      if (t.nd != 3 || t.dims[2] != (uint64_t)ne || t.dims[1] != rows || t.dims[0] != cols)
        return llb_fail_msg(LLB_HIP_EINVAL, ("table: " + nm + ": an expert stack of the wrong shape").c_str());
      if (t.type != 8 && t.type != 12 && t.type != 13 && t.type != 14)
        return llb_fail_msg(LLB_HIP_EINVAL, ("table: " + nm + ": expert stacks take Q8_0, Q4_K, Q5_K, Q6_K").c_str());
    }
    w[26] |= fm << (4 * x) | (fz ? 1u << 12 : 0u) | 1u << 13;
  }
  for (uint32_t L = 0; L < nl; L++) {
    const uint8_t* r = &need[L * 6];
    if (!r[0] || !r[1] || !r[5] || (!r[4] && (!r[2] || !r[3])) || (r[4] && (r[2] || r[3])))
      return llb_fail_msg(LLB_HIP_EINVAL, "table: a layer without its router, shared gate or expert stacks");
    uint32_t* w = table + L * 32;
    if (w[26] >> 12 & 1) w[26] |= (w[26] & 15) << 4;  // fused: up has gate's format
    w[27] = (uint32_t)ne;
    w[28] = (uint32_t)ef;
    w[29] = (uint32_t)sf;
    w[30] = (uint32_t)nk;
  }
  return 0;
}

int llb_gguf_find(const llb_gguf* g, const char* name) {
  if (!g || !name) return -1;
  for (size_t i = 0; i < g->t.size(); i++)
    if (g->t[i].name == name) return (int)i;
  return -1;
}

}  // extern "C"

// one stack's bytes into its residency (moe_fill, host/llb_host.c:445-487)
static int fill(const llb_gguf* g, const GgTensor& t, int mode, llb_dptr* out, const char* what) {
  char msg[256];
  if (mode == LLB_MOE_RES_HOST) {
    void* h = nullptr;
    if (hipHostMalloc(&h, t.bytes, hipHostMallocMapped | hipHostMallocPortable) != hipSuccess) {
      snprintf(msg, sizeof msg, "gguf: cannot pin %llu bytes of host memory for %s", (unsigned long long)t.bytes, what);
      return llb_fail_msg(LLB_HIP_EDEVICE, msg);
    }
    for (uint64_t k = 0; k < t.bytes;) {
      const uint64_t c = t.bytes - k > (1ull << 30) ? (1ull << 30) : t.bytes - k;
      const ssize_t r = pread(g->fd, (uint8_t*)h + k, (size_t)c, (off_t)(t.off + k));
      if (r <= 0) {
        (void)hipHostFree(h);
        return llb_fail_msg(LLB_HIP_EINVAL, "gguf: read failed");
      }
      k += (uint64_t)r;
    }
    void* dp = nullptr;
    if (hipHostGetDevicePointer(&dp, h, 0) != hipSuccess) {
      (void)hipHostFree(h);
      return llb_fail_msg(LLB_HIP_EDEVICE, "gguf: no device address for the pinned stack");
    }
    *out = (llb_dptr)(uintptr_t)dp;
    return 0;
  }
  void* d = nullptr;
  if (hipMalloc(&d, t.bytes) != hipSuccess) {
    snprintf(msg, sizeof msg, "gguf: cannot allocate %llu bytes of device memory for %s", (unsigned long long)t.bytes, what);
    return llb_fail_msg(LLB_HIP_EDEVICE, msg);
  }
  const uint64_t CH = 64ull << 20;
  void* buf = nullptr;
  if (hipHostMalloc(&buf, CH, 0) != hipSuccess) {
    (void)hipFree(d);
    return llb_fail_msg(LLB_HIP_EDEVICE, "gguf: cannot pin the upload buffer");
  }
  int rc = 0;
  for (uint64_t k = 0; k < t.bytes && !rc; k += CH) {
    const uint64_t c = t.bytes - k < CH ? t.bytes - k : CH;
    for (uint64_t q = 0; q < c;) {
      const ssize_t r = pread(g->fd, (uint8_t*)buf + q, (size_t)(c - q), (off_t)(t.off + k + q));
      if (r <= 0) {
        rc = llb_fail_msg(LLB_HIP_EINVAL, "gguf: read failed");
        break;
      }
      q += (uint64_t)r;
    }
    if (!rc && hipMemcpy((uint8_t*)d + k, buf, c, hipMemcpyHostToDevice) != hipSuccess)
      rc = llb_fail_msg(LLB_HIP_EDEVICE, "gguf: cannot upload a stack");
  }
  (void)hipHostFree(buf);
  if (rc) {
    (void)hipFree(d);
    return rc;
  }
  *out = (llb_dptr)(uintptr_t)d;
  return 0;
}

static void free_stack(int mode, llb_dptr p) {
  if (!p) return;
  if (mode == LLB_MOE_RES_HOST) {
    hipPointerAttribute_t a;
    void* h = (hipPointerGetAttributes(&a, (void*)(uintptr_t)p) == hipSuccess && a.hostPointer) ? a.hostPointer
                                                                                            : (void*)(uintptr_t)p;
    (void)hipHostFree(h);
  } else {
    (void)hipFree((void*)(uintptr_t)p);
  }
}

// a named tensor of the layer with its expected format and bytes (the reference's check against the
// sidecar, host/llb_host.c:509-515)
static const GgTensor* want(const llb_gguf* g, uint32_t layer, const char* nm, uint32_t fm, uint64_t bytes, int* rc) {
  char name[96], msg[256];
  snprintf(name, sizeof name, "blk.%u.%s.weight", layer, nm);
  const int i = llb_gguf_find(g, name);
  if (i < 0) {
    snprintf(msg, sizeof msg, "gguf: %s not found", name);
    *rc = llb_fail_msg(LLB_HIP_EINVAL, msg);
    return nullptr;
  }
  const GgTensor& t = g->t[(size_t)i];
  if (gg_fm(t.type) != (int)fm || t.bytes != bytes) {
    snprintf(msg, sizeof msg, "gguf: %s: ggml type %u, %llu bytes; the layer says format %u, %llu bytes", name, t.type,
             (unsigned long long)t.bytes, fm, (unsigned long long)bytes);
    *rc = llb_fail_msg(LLB_HIP_EINVAL, msg);
    return nullptr;
  }
  return &t;
}

// per-layer stream state: the mapped file and the staging for k experts (llb_moe_load's mode 2)
struct StreamSrc {
  const uint8_t* map;
  uint64_t map_bytes;
  uint64_t sg, su, sd;  // stack offsets in the file
  uint64_t esg, esd;    // expert strides of the gate (and up) and down stacks
  bool fused;
  void* pin;            // pinned host staging, nk experts
  void* dev;            // device staging: nk gate (+ up) experts, then nk down experts
  uint32_t* slots;      // device [nk] = 0 .. nk - 1: the ids the expert kernels see
  uint32_t nk;
};
static void free_stream(StreamSrc* s) {
  if (!s) return;
  (void)hipStreamSynchronize(llb_cur_stream());
  (void)hipHostFree(s->pin);
  (void)hipFree(s->dev);
  (void)hipFree(s->slots);
  munmap((void*)s->map, (size_t)s->map_bytes);
  delete s;
}

extern "C" {

static int load_layer_impl(llb_gguf* g, uint32_t layer, int mode, llb_moe_layer* L) {
  if (!g || !L) return llb_fail_msg(LLB_HIP_EINVAL, "load: null file or layer");
  if (mode < LLB_MOE_RES_DEVICE || mode > LLB_MOE_RES_STREAM) return llb_fail_msg(LLB_HIP_EINVAL, "load: no such mode");
  const uint32_t fg = L->fx & 15, fu = L->fx >> 4 & 15, fd = L->fx >> 8 & 15, fz = L->fx >> 12 & 1;
  const uint64_t rbg = row_bytes(fg, L->dm), rbu = row_bytes(fu, L->dm), rbd = row_bytes(fd, L->ef);
  if (!L->dm || !L->ne || !L->ef || !L->nk || !rbg || !rbu || !rbd) return llb_fail_msg(LLB_HIP_EINVAL, "load: the layer's shape words are not set");
  int rc = 0;
  const GgTensor* tg = want(g, layer, fz ? "ffn_gate_up_exps" : "ffn_gate_exps", fg,
                            (uint64_t)L->ne * (fz ? 2 : 1) * L->ef * rbg, &rc);
  if (!tg) return rc;
  const GgTensor* tu = nullptr;
  if (!fz && !(tu = want(g, layer, "ffn_up_exps", fu, (uint64_t)L->ne * L->ef * rbu, &rc))) return rc;
  const GgTensor* td = want(g, layer, "ffn_down_exps", fd, (uint64_t)L->ne * L->dm * rbd, &rc);
  if (!td) return rc;
  // router, shared gate row and shared expert, when the caller has not placed them
  struct Opt {
    const char* nm;
    llb_dptr* dst;
    uint32_t fm;
    uint64_t bytes;
  } opt[5] = {
      {"ffn_gate_inp", &L->router, LLB_FM_F32, (uint64_t)L->ne * L->dm * 4},
      {"ffn_gate_inp_shexp", &L->shgate, LLB_FM_F32, (uint64_t)L->dm * 4},
      {"ffn_gate_shexp", &L->SG, L->fsg, (uint64_t)L->sf * row_bytes(L->fsg, L->dm)},
      {"ffn_up_shexp", &L->SU, L->fsu, (uint64_t)L->sf * row_bytes(L->fsu, L->dm)},
      {"ffn_down_shexp", &L->SD, L->fsd, (uint64_t)L->dm * row_bytes(L->fsd, L->sf)},
  };
  const GgTensor* ot[5] = {};
  for (int i = 0; i < 5; i++) {
    if (*opt[i].dst || (i >= 1 && !L->sf)) continue;
    char name[96];
    snprintf(name, sizeof name, "blk.%u.%s.weight", layer, opt[i].nm);
    if (llb_gguf_find(g, name) < 0) continue;  // the caller supplies it
    if (!(ot[i] = want(g, layer, opt[i].nm, opt[i].fm, opt[i].bytes, &rc))) return rc;
  }
  llb_dptr got[3] = {0, 0, 0};
  const GgTensor* st[3] = {tg, tu, td};
  if (mode == LLB_MOE_RES_STREAM) {
    struct stat sb;
    if (fstat(g->fd, &sb) != 0) return llb_fail_msg(LLB_HIP_EINVAL, "load: cannot stat the file");
    void* map = mmap(nullptr, (size_t)sb.st_size, PROT_READ, MAP_SHARED, g->fd, 0);
    if (map == MAP_FAILED) return llb_fail_msg(LLB_HIP_EINVAL, "load: cannot map the file");
    auto* s = new StreamSrc{};
    s->map = (const uint8_t*)map;
    s->map_bytes = (uint64_t)sb.st_size;
    s->sg = tg->off;
    s->su = tu ? tu->off : tg->off + (uint64_t)L->ef * rbg;
    s->sd = td->off;
    s->fused = fz;
    s->esg = (uint64_t)(fz ? 2 : 1) * L->ef * rbg;
    s->esd = (uint64_t)L->dm * rbd;
    s->nk = L->nk;
    const uint64_t ex = (fz ? s->esg : 2 * (uint64_t)L->ef * rbg) + s->esd;  // one expert's bytes
    std::vector<uint32_t> sl(L->nk);
    for (uint32_t j = 0; j < L->nk; j++) sl[j] = j;
    if (hipHostMalloc(&s->pin, ex * L->nk, 0) != hipSuccess || hipMalloc(&s->dev, ex * L->nk) != hipSuccess ||
        hipMalloc((void**)&s->slots, 4ull * L->nk) != hipSuccess ||
        hipMemcpy(s->slots, sl.data(), 4ull * L->nk, hipMemcpyHostToDevice) != hipSuccess) {
      if (s->pin) (void)hipHostFree(s->pin);
      if (s->dev) (void)hipFree(s->dev);
      if (s->slots) (void)hipFree(s->slots);
      munmap(map, (size_t)sb.st_size);
      delete s;
      return llb_fail_msg(LLB_HIP_EDEVICE, "load: cannot allocate the stream staging");
    }
    L->stream = (llb_dptr)(uintptr_t)s;
    // G / U / D: the device staging slots (gate of slot j at j esg-with-up-or-not, see the forward)
    const uint64_t gb = fz ? s->esg : (uint64_t)L->ef * rbg;
    got[0] = (llb_dptr)(uintptr_t)s->dev;
    got[1] = fz ? 0 : got[0] + gb * L->nk;
    got[2] = got[0] + (fz ? s->esg : 2 * gb) * L->nk;
  } else {
    for (int i = 0; i < 3; i++)
      if (st[i] && (rc = fill(g, *st[i], mode, &got[i], i == 0 ? "a gate stack" : i == 1 ? "an up stack" : "a down stack"))) {
        for (int k = 0; k < i; k++) free_stack(mode, got[k]);
        return rc;
      }
  }
  uint32_t own = 0;
  for (int i = 0; i < 5; i++)
    if (ot[i]) {
      if ((rc = fill(g, *ot[i], LLB_MOE_RES_DEVICE, opt[i].dst, opt[i].nm))) {
        // unwind: the optional tensors filled so far, then the stacks or the stream state
        for (int k = 0; k < i; k++)
          if (own >> k & 1) {
            free_stack(LLB_MOE_RES_DEVICE, *opt[k].dst);
            *opt[k].dst = 0;
          }
        if (mode == LLB_MOE_RES_STREAM) {
          free_stream((StreamSrc*)(uintptr_t)L->stream);
          L->stream = 0;
        } else {
          for (int k = 0; k < 3; k++) free_stack(mode, got[k]);
        }
        return rc;
      }
      own |= 1u << i;
    }
  L->G = got[0];
  L->U = fz ? 0 : got[1];
  L->D = got[2];
  L->res = (uint32_t)mode;
  L->own = own;
  return 0;
}
int llb_moe_hip_load_layer(llb_gguf* g, uint32_t layer, int mode, llb_moe_layer* L) {
  try {
    return load_layer_impl(g, layer, mode, L);
  } catch (...) {  // a bad_alloc of the stream state: nothing crosses the C ABI
    return llb_fail_msg(LLB_HIP_EDEVICE, "load: out of host memory");
  }
}

// llb_moe_load's residency choice (host/llb_host.c:532-545): the routed experts' bytes over the n layers
// (each stack checked against the file as load_layer checks it), against free device memory less a
// 0.75 GiB reserve (device), then MemAvailable less 4 GiB (host), else stream. LLB_MOE_VRAM / LLB_MOE_RAM
// (bytes) stand in for the two capacities, LLB_MOE_EXPERTS=device|host|stream forces the mode; one line
// on stderr names the choice and its inputs.
static uint64_t env_bytes(const char* k, bool* set) {
  const char* e = getenv(k);
  *set = e && *e;
  return *set ? strtoull(e, nullptr, 10) : 0;
}
static uint64_t mem_available() {
  FILE* f = fopen("/proc/meminfo", "r");
  if (!f) return 0;
  char ln[256];
  uint64_t kb = 0;
  while (fgets(ln, sizeof ln, f))
    if (!strncmp(ln, "MemAvailable:", 13)) kb = strtoull(ln + 13, nullptr, 10);
  fclose(f);
  return kb * 1024;
}
int llb_moe_hip_residency(const llb_gguf* g, const uint32_t* layers, const llb_moe_layer* L, uint32_t n, int* mode,
                          uint64_t* expert_bytes) {
  if (!g || !layers || !L || !mode || !n) return llb_fail_msg(LLB_HIP_EINVAL, "residency: null argument or no layers");
  uint64_t tot = 0;
  int rc = 0;
  for (uint32_t i = 0; i < n; i++) {
    const llb_moe_layer& l = L[i];
    const uint32_t fg = l.fx & 15, fu = l.fx >> 4 & 15, fd = l.fx >> 8 & 15, fz = l.fx >> 12 & 1;
    const uint64_t rbg = row_bytes(fg, l.dm), rbu = row_bytes(fu, l.dm), rbd = row_bytes(fd, l.ef);
    if (!l.dm || !l.ne || !l.ef || !rbg || !rbu || !rbd)
      return llb_fail_msg(LLB_HIP_EINVAL, "residency: a layer's shape words are not set");
    const GgTensor* t = want(g, layers[i], fz ? "ffn_gate_up_exps" : "ffn_gate_exps", fg,
                             (uint64_t)l.ne * (fz ? 2 : 1) * l.ef * rbg, &rc);
    if (!t) return rc;
    tot += t->bytes;
    if (!fz) {
      if (!(t = want(g, layers[i], "ffn_up_exps", fu, (uint64_t)l.ne * l.ef * rbu, &rc))) return rc;
      tot += t->bytes;
    }
    if (!(t = want(g, layers[i], "ffn_down_exps", fd, (uint64_t)l.ne * l.dm * rbd, &rc))) return rc;
    tot += t->bytes;
  }
  bool vset, rset;
  uint64_t vram = env_bytes("LLB_MOE_VRAM", &vset), ram = env_bytes("LLB_MOE_RAM", &rset);
  if (!vset) {
    size_t fr = 0, tv = 0;
    if (hipMemGetInfo(&fr, &tv) != hipSuccess) {
      (void)hipGetLastError();
      return llb_fail_msg(LLB_HIP_EDEVICE, "residency: hipMemGetInfo failed (set LLB_MOE_VRAM to choose without a device)");
    }
    vram = fr;
  }
  if (!rset) ram = mem_available();
  const uint64_t rv = 3ull << 28, rr = 4ull << 30;
  const char* e = getenv("LLB_MOE_EXPERTS");
  int m;
  if (e && !strcmp(e, "device")) m = LLB_MOE_RES_DEVICE;
  else if (e && !strcmp(e, "host")) m = LLB_MOE_RES_HOST;
  else if (e && !strcmp(e, "stream")) m = LLB_MOE_RES_STREAM;
  else m = tot + rv <= vram ? LLB_MOE_RES_DEVICE : tot + rr <= ram ? LLB_MOE_RES_HOST : LLB_MOE_RES_STREAM;
  static const char* mn[3] = {"device (VRAM)", "host (pinned, device-mapped RAM)",
                              "stream (mmapped GGUF, the k experts copied per token)"};
  fprintf(stderr, "moe: %u layers, experts %.2f GiB -> %s [free VRAM %.2f GiB%s, MemAvailable %.2f GiB%s]\n", n,
          tot / 1073741824.0, mn[m], vram / 1073741824.0, vset ? " (LLB_MOE_VRAM)" : "", ram / 1073741824.0,
          rset ? " (LLB_MOE_RAM)" : "");
  *mode = m;
  if (expert_bytes) *expert_bytes = tot;
  return 0;
}

}  // extern "C"

// The stream gather's worker pool (the reference spreads the per-token copy over 8 threads,
// host/llb_host.c:680-696). One pool a process, made on its first streamed token and never torn down:
// its threads sleep on the condition variable between tokens, and at exit the process ends them. The
// calling thread is worker 0. A job is a list of source segments laid end to end in dst; the bytes
// [0, total) are cut into kGather equal pieces, piece i copied by worker i. run() returns when every
// piece is copied, and the mutex orders those writes before the caller's upload.
namespace {
constexpr unsigned kGather = 8;
struct Seg {
  const uint8_t* src;
  uint64_t len;
};
struct GatherPool {
  std::mutex call;  // one job at a time: callers on several threads queue here
  std::mutex m;
  std::condition_variable go, done;
  uint64_t gen = 0;
  unsigned left = 0;
  const Seg* seg = nullptr;
  size_t nseg = 0;
  uint64_t total = 0;
  uint8_t* dst = nullptr;
  void piece(unsigned i) {
    const uint64_t lo = total * i / kGather, hi = total * (i + 1) / kGather;
    uint64_t base = 0;
    for (size_t k = 0; k < nseg && base < hi; base += seg[k++].len) {
      const uint64_t a = lo > base ? lo : base, b = hi < base + seg[k].len ? hi : base + seg[k].len;
      if (a < b) memcpy(dst + a, seg[k].src + (a - base), b - a);
    }
  }
  void worker(unsigned i) {
    uint64_t seen = 0;
    for (;;) {
      {
        std::unique_lock<std::mutex> lk(m);
        go.wait(lk, [&] { return gen != seen; });
        seen = gen;
      }
      piece(i);
      std::lock_guard<std::mutex> lk(m);
      if (--left == 0) done.notify_one();
    }
  }
  void run(uint8_t* d, const std::vector<Seg>& sv) {
    std::lock_guard<std::mutex> one(call);
    {
      std::lock_guard<std::mutex> lk(m);
      dst = d, seg = sv.data(), nseg = sv.size(), total = 0;
      for (const Seg& x : sv) total += x.len;
      left = kGather - 1;
      gen++;
    }
    go.notify_all();
    piece(0);
    std::unique_lock<std::mutex> lk(m);
    done.wait(lk, [&] { return left == 0; });
  }
};
// the pool of this process: a child made by fork() inherits the pool's memory but not its threads, so
// a pool made by another process id is left behind (never touched again) and a new one is made
// A pool that cannot be made (no memory, a thread limit) is not an error: the caller copies on its own
// thread instead, and this process does not try again. No exception leaves this function, so none reaches
// the C entry points above it.
GatherPool* gather_pool() {
  static std::mutex mk;
  static GatherPool* p = nullptr;
  static pid_t owner = 0;
  static bool broken = false;
  std::lock_guard<std::mutex> lk(mk);
  if (!p || owner != getpid()) {
    if (broken && owner == getpid()) return nullptr;
    owner = getpid();
    p = new (std::nothrow) GatherPool;  // never freed: detached workers wait on it until the process ends
    unsigned made = 1;
    if (p) {
      try {
        for (; made < kGather; made++) std::thread(&GatherPool::worker, p, made).detach();
      } catch (...) {
      }
    }
    if (!p || made < kGather) {  // the workers made so far keep waiting on the abandoned pool
      p = nullptr;
      broken = true;
    }
  }
  return p;
}
// the same job on the calling thread
void gather_here(uint8_t* dst, const std::vector<Seg>& sv) {
  for (const Seg& g : sv) {
    memcpy(dst, g.src, g.len);
    dst += g.len;
  }
}
}  // namespace

// the k chosen experts of one token into the device staging (the reference's per-token copy,
// host/llb_host.c:680-696): ids read back, the experts' gate (+ up) and down bytes gathered from the
// mapped file into pinned memory by the pool, then uploaded on the library stream. The slot ids 0..k-1
// replace the experts' ids for the expert kernels.
static int stream_stage_impl(const llb_moe_layer* L, const uint32_t* d_ids, const uint32_t** slots) {
  auto* s = (StreamSrc*)(uintptr_t)L->stream;
  if (!s) return llb_fail_msg(LLB_HIP_EINVAL, "stream: the layer has no stream source");
  const hipStream_t st = llb_cur_stream();
  std::vector<uint32_t> ids(s->nk);
  if (hipMemcpyAsync(ids.data(), d_ids, 4ull * s->nk, hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return llb_fail_msg(LLB_HIP_EDEVICE, "stream: cannot read the chosen experts back");
  const uint64_t gb = s->esg, ub = s->fused ? 0 : s->esg, db = s->esd;
  uint8_t* pin = (uint8_t*)s->pin;
  uint8_t* dev = (uint8_t*)s->dev;
  for (uint32_t j = 0; j < s->nk; j++)
    if (ids[j] >= L->ne) return llb_fail_msg(LLB_HIP_EINVAL, "stream: an expert id out of range");
  // gathered in the device staging's order (the nk gate experts, the nk up experts, the nk down experts),
  // one job and one upload a stack: the pool gathers a stack while the copy engine uploads the one before
  GatherPool* pool = gather_pool();
  std::vector<Seg> sv;
  sv.reserve(s->nk);
  const uint64_t base[3] = {s->sg, s->su, s->sd}, es[3] = {s->esg, s->esg, s->esd}, len[3] = {gb, ub, db};
  uint64_t at = 0;
  for (int k = 0; k < 3; k++) {
    if (!len[k]) continue;  // fused stacks: the up rows travel with the gate rows
    sv.clear();
    for (uint32_t j = 0; j < s->nk; j++) sv.push_back({s->map + base[k] + ids[j] * es[k], len[k]});
    if (pool) pool->run(pin + at, sv);
    else gather_here(pin + at, sv);
    if (hipMemcpyAsync(dev + at, pin + at, s->nk * len[k], hipMemcpyHostToDevice, st) != hipSuccess)
      return llb_fail_msg(LLB_HIP_EDEVICE, "stream: cannot stage the experts");
    at += s->nk * len[k];
  }
  *slots = s->slots;
  return 0;
}
// no exception (a vector's bad_alloc) crosses into the C entry point that calls this
int stream_stage(const llb_moe_layer* L, const uint32_t* d_ids, const uint32_t** slots) {
  try {
    return stream_stage_impl(L, d_ids, slots);
  } catch (...) {
    return llb_fail_msg(LLB_HIP_EDEVICE, "stream: out of host memory staging the experts");
  }
}
// the pinned staging is reused by the next token: wait for this token's uploads (the caller, after
// the expert kernels are queued)
int stream_done() {
  return hipStreamSynchronize(llb_cur_stream()) == hipSuccess ? 0 : llb_fail_msg(LLB_HIP_EDEVICE, "stream: sync");
}

extern "C" int llb_moe_hip_unload_layer(llb_moe_layer* L) {
  if (!L) return llb_fail_msg(LLB_HIP_EINVAL, "unload: null layer");
  if (L->res == LLB_MOE_RES_STREAM) {
    free_stream((StreamSrc*)(uintptr_t)L->stream);
    L->stream = 0;
  } else {
    free_stack((int)L->res, L->G);
    free_stack((int)L->res, L->U);
    free_stack((int)L->res, L->D);
  }
  llb_dptr* opt[5] = {&L->router, &L->shgate, &L->SG, &L->SU, &L->SD};
  for (int i = 0; i < 5; i++)
    if (L->own >> i & 1) {
      free_stack(LLB_MOE_RES_DEVICE, *opt[i]);
      *opt[i] = 0;
    }
  L->own = 0;
  L->G = L->U = L->D = 0;
  return 0;
}
