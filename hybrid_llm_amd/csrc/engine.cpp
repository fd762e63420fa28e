// Native engine behind the reference's engine C API (llmy_cuda/include/llmy.h:31-72):
// llmy_load / llmy_free, introspection, state handles, llmy_prefill,
// llmy_decode, llmy_sample, llmy_last_executed_loops, llmy_sync, plus batched
// forms of prefill/decode and a status query.
//
// The model handle owns the device weights, the state handle the per
// (loop, layer) KV caches, GDN states and conv histories and every
// activation buffer, as the reference's Model and State do
// (llmy_cuda/include/model.h:143-267).  The reference engine is batch-1 and
// fp32 (llmy_cuda/src/model.cpp:627); this one runs B sequences per state in
// bf16 through the same kernels as hybrid_llm_amd/engine.py:
//   decode  = embedding + pre-norm, then per (loop, layer) the attention or GDN
//             mixer and the MoE (fused router, route-indexed experts, combine
//             fused with the next pre-norm), the tied LM head;
//   prefill = the same blocks over all B*T prompt tokens with the sequence
//             kernels (banded attention prefill + KV ring fill, GDN input
//             preparation + chunked scan + output gate + sequence conv gate,
//             router + permutation + grouped expert GEMMs), from position 0.
// Weights come from a `.llmy` v1 file (format of
// llmy_cuda/tools/convert_checkpoint.py:1-31; parsed here with bounds checks
// on every index entry) through mmap.
//
// No C++ exception leaves the C ABI: each entry point catches, records the
// message (llmy_last_status / llmy_last_error) and returns NULL or a nonzero
// status, where the reference would have let a throw escape
// (llmy_cuda/src/llmy.cpp:116-131).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "llmy.h"

namespace {

thread_local int32_t g_status = 0;
thread_local char g_error[512] = "";

void set_error(int32_t st, const char* msg) {
  g_status = st;
  std::snprintf(g_error, sizeof(g_error), "%s", msg);
}

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess)
    throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void check_call(int32_t st, const char* what) {
  if (st != 0) throw std::runtime_error(std::string(what) + " returned status " + std::to_string(st));
}

// ------------------------------------------------------------------ .llmy reader
constexpr uint32_t kVersion = 1;
constexpr size_t kEntry = 108;
constexpr size_t kAlign = 4096;

struct TensorRef {
  uint32_t dtype = 0;  // 0 f32, 1 f16, 2 bf16
  std::vector<int64_t> shape;
  const unsigned char* data = nullptr;
  uint64_t nbytes = 0;
  int64_t numel() const {
    int64_t n = 1;
    for (int64_t s : shape) n *= s;
    return n;
  }
};

struct MappedFile {
  void* base = MAP_FAILED;
  size_t size = 0;
  ~MappedFile() {
    if (base != MAP_FAILED) munmap(base, size);
  }
};

struct Checkpoint {
  MappedFile file;
  std::string config;
  std::map<std::string, TensorRef> tensors;

  const TensorRef& get(const std::string& name) const {
    auto it = tensors.find(name);
    if (it == tensors.end()) throw std::runtime_error("checkpoint has no tensor " + name);
    return it->second;
  }
};

template <typename T>
T read_le(const unsigned char* p) {
  T v;
  std::memcpy(&v, p, sizeof(T));
  return v;
}

void parse_checkpoint(const char* path, Checkpoint& ck) {
  const int fd = open(path, O_RDONLY);
  if (fd < 0) throw std::runtime_error(std::string("cannot open ") + path);
  struct stat st {};
  if (fstat(fd, &st) != 0) {
    close(fd);
    throw std::runtime_error("cannot stat checkpoint");
  }
  ck.file.size = static_cast<size_t>(st.st_size);
  ck.file.base = ck.file.size ? mmap(nullptr, ck.file.size, PROT_READ, MAP_PRIVATE, fd, 0) : MAP_FAILED;
  close(fd);
  if (ck.file.base == MAP_FAILED) throw std::runtime_error("cannot map checkpoint");
  const auto* b = static_cast<const unsigned char*>(ck.file.base);
  const size_t n = ck.file.size;
  if (n < 16 || std::memcmp(b, "LLMY", 4) != 0) throw std::runtime_error("bad magic");
  if (read_le<uint32_t>(b + 4) != kVersion) throw std::runtime_error("unsupported version");
  const uint64_t cfg_len = read_le<uint32_t>(b + 8);
  if (12 + cfg_len + 4 > n) throw std::runtime_error("truncated config");
  ck.config.assign(reinterpret_cast<const char*>(b + 12), cfg_len);
  const uint64_t count = read_le<uint32_t>(b + 12 + cfg_len);
  const uint64_t index = 16 + cfg_len;
  const uint64_t index_end = index + count * kEntry;
  if (index_end > n) throw std::runtime_error("truncated index");
  const uint64_t data_start = (index_end + kAlign - 1) / kAlign * kAlign;
  for (uint64_t i = 0; i < count; ++i) {
    const unsigned char* e = b + index + i * kEntry;
    const uint32_t name_len = read_le<uint32_t>(e);
    if (name_len > 63) throw std::runtime_error("bad tensor name length");
    TensorRef t;
    std::string name(reinterpret_cast<const char*>(e + 4), name_len);
    t.dtype = read_le<uint32_t>(e + 68);
    const uint32_t ndim = read_le<uint32_t>(e + 72);
    if (t.dtype > 2 || ndim > 4) throw std::runtime_error("bad dtype or rank for " + name);
    for (uint32_t d = 0; d < ndim; ++d) t.shape.push_back(read_le<uint32_t>(e + 76 + 4 * d));
    const uint64_t off = read_le<uint64_t>(e + 92);
    t.nbytes = read_le<uint64_t>(e + 100);
    const uint64_t item = t.dtype == 0 ? 4 : 2;
    if (t.nbytes != static_cast<uint64_t>(t.numel()) * item)
      throw std::runtime_error("size does not match shape for " + name);
    if (data_start > n || off > n - data_start || t.nbytes > n - data_start - off)
      throw std::runtime_error("payload outside the file for " + name);
    t.data = b + data_start + off;
    ck.tensors[name] = t;
  }
}

std::map<std::string, std::string> parse_config(const std::string& text) {
  std::map<std::string, std::string> kv;
  size_t p = 0;
  while (p < text.size()) {
    size_t e = text.find('\n', p);
    if (e == std::string::npos) e = text.size();
    const std::string line = text.substr(p, e - p);
    const size_t eq = line.find('=');
    if (eq != std::string::npos) kv[line.substr(0, eq)] = line.substr(eq + 1);
    p = e + 1;
  }
  return kv;
}

// ------------------------------------------------------------------ model
enum Kind { kAttn = 0, kGdn = 1, kCsa = 2, kHca = 3 };

// Heads, head width, local window, compression ratio and top-k (0 = dense) of
// a compressed-memory mixer (model/model.py:95-106).
struct CmpShape {
  int H = 0, Dh = 0, W = 0, ratio = 0, top_k = 0;
  int kw() const { return H * Dh; }
};

struct Config {
  int vocab = 0, d_model = 0, num_loops = 0;
  std::vector<int> kinds;
  int attn_heads = 0, attn_head_dim = 0, window = 0;
  int gdn_heads = 0, dk = 0, dv = 0, conv_kernel = 4;
  int experts = 0, top_k = 0, hidden = 0;
  int shared = 0;  // shared experts, stacked after the routed ones (experts .. experts+shared-1)
  // context-aware router (local latent window): router.context_aware,
  // router.local_context, mla.latent_dim (llmy_cuda/include/config.h:60-66)
  bool ctx = false;
  int ctx_window = 128, latent = 256;
  // the router's global branch on HCA blocks: latent attention with
  // router.query_heads x router.query_head_dim (llmy_cuda/include/config.h)
  int router_heads = 4, router_head_dim = 64;
  int hq() const { return router_heads * router_head_dim; }
  // multi-stream hyper-connections: streams per token (mhc.streams when
  // mhc.enabled; 1 = the single residual stream) and Sinkhorn iterations
  int mhc = 1, mhc_iters = 20;
  // compressed-memory mixers: csa.* / hca.* keys (llmy_cuda/include/config.h:41-51)
  // and the decode memory's slots per row (memory.decode_slots; the reference
  // native engine's fixed 256, llmy_cuda/src/model.cpp:351-354)
  int csa_heads = 16, csa_head_dim = 128, csa_window = 128, csa_ratio = 4, csa_top_k = 32;
  int hca_window = 128, hca_ratio = 32, hca_top_k = 32;
  bool hca_dense = true;
  int cmp_slots = 256;
  // stem / tail blocks (GDN + dense SwiGLU FFN of width dense_hidden,
  // model/model.py:391-394,411-414): stem_blocks, tail_blocks, dense_ffn.hidden
  int stem = 0, tail = 0, dense_hidden = 0;
  float eps = 1e-6f;
  // widths as the GEMM kernels take them: zero-padded to a multiple of 256
  static int pad256(int n) { return (n + 255) / 256 * 256; }
  int hidden_p() const { return pad256(hidden); }
  int dense_p() const { return pad256(dense_hidden); }
  int latent_p() const { return pad256(latent); }
  int hq_p() const { return pad256(hq()); }
  bool has_gdn() const { return has(kGdn) || stem > 0 || tail > 0; }
  CmpShape cmp(int kind) const {
    CmpShape c;
    if (kind == kCsa) {
      c.H = csa_heads, c.Dh = csa_head_dim, c.W = csa_window, c.ratio = csa_ratio;
      c.top_k = csa_top_k;
    } else {
      c.H = 1, c.Dh = d_model, c.W = hca_window, c.ratio = hca_ratio;
      c.top_k = hca_dense ? 0 : hca_top_k;
    }
    return c;
  }
  bool has(int kind) const { return std::count(kinds.begin(), kinds.end(), kind) > 0; }
  int mhc_n16() const { return (2 * mhc + mhc * mhc + 15) / 16 * 16; }
  int routes() const { return top_k + shared; }      // routes per token, shared included
  int all_experts() const { return experts + shared; }
  int nproj16() const {
    const int n = 2 * gdn_heads * dk + 2 * gdn_heads * dv + gdn_heads;
    return (n + 15) / 16 * 16;
  }
};

int cfg_int(const std::map<std::string, std::string>& kv, const char* key, int dflt, bool need) {
  auto it = kv.find(key);
  if (it == kv.end()) {
    if (need) throw std::runtime_error(std::string("config lacks ") + key);
    return dflt;
  }
  return std::stoi(it->second);
}

// Boolean config values as the reference reads them (llmy_cuda/src/config.cpp:18-22).
bool cfg_bool(const std::map<std::string, std::string>& kv, const char* key, bool dflt) {
  auto it = kv.find(key);
  if (it == kv.end()) return dflt;
  const std::string& v = it->second;
  if (v == "1" || v == "true" || v == "True" || v == "yes") return true;
  if (v == "0" || v == "false" || v == "False" || v == "no") return false;
  throw std::runtime_error(std::string("expected bool for ") + key);
}

Config config_from(const std::string& text) {
  const auto kv = parse_config(text);
  Config c;
  c.vocab = cfg_int(kv, "vocab_size", 0, true);
  c.d_model = cfg_int(kv, "d_model", 0, true);
  c.num_loops = cfg_int(kv, "num_loops", 1, true);
  c.stem = cfg_int(kv, "stem_blocks", 0, false);
  c.tail = cfg_int(kv, "tail_blocks", 0, false);
  c.dense_hidden = cfg_int(kv, "dense_ffn.hidden", 3584, false);
  // keys that change the reference model's math in ways this engine does not
  // run are refused rather than ignored
  if (cfg_bool(kv, "loop_attnres.enabled", false))
    throw std::runtime_error("loop_attnres.enabled: the loop-attention residual "
                             "(model/loop_memory.py) is not part of this engine");
  if (cfg_bool(kv, "adaptive_loops.enabled", false))
    throw std::runtime_error("adaptive_loops.enabled: learned halting is not part of this "
                             "engine; run a fixed loop count");
  if (!cfg_bool(kv, "mhc.shared_across_loops", true))
    throw std::runtime_error("mhc.shared_across_loops = 0: per-loop block copies "
                             "(model.py:397-408) are not part of this engine");
  if (!cfg_bool(kv, "mhc.preserve_streams_across_loop_boundary", true))
    throw std::runtime_error("mhc.preserve_streams_across_loop_boundary = 0: the per-loop "
                             "stream reset (model.py:634-635) is not part of this engine");
  // mHC keys with the reference's defaults (llmy_cuda/include/config.h:27-29)
  if (cfg_bool(kv, "mhc.enabled", true)) {
    c.mhc = cfg_int(kv, "mhc.streams", 4, false);
    c.mhc_iters = cfg_int(kv, "mhc.sinkhorn_iterations", 20, false);
    if (c.mhc != 2 && c.mhc != 4) throw std::runtime_error("mhc.streams must be 2 or 4");
  } else if (cfg_int(kv, "mhc.streams", 1, false) != 1) {
    throw std::runtime_error("streams without mHC maps (mhc.enabled = 0, mhc.streams > 1) "
                             "are not part of this engine");
  }
  auto lay = kv.find("recurrent_layout");
  if (lay == kv.end()) throw std::runtime_error("config lacks recurrent_layout");
  size_t p = 0;
  const std::string& s = lay->second;
  while (p <= s.size()) {
    size_t e = s.find(',', p);
    if (e == std::string::npos) e = s.size();
    std::string k = s.substr(p, e - p);
    // every core block carries a MoE: "gdn_moe" and "gdn" name the same block
    // (the mixer kind is the part before '_', model/model.py:395)
    if (k.size() > 4 && k.compare(k.size() - 4, 4, "_moe") == 0) k.resize(k.size() - 4);
    if (k == "attn") c.kinds.push_back(kAttn);
    else if (k == "gdn") c.kinds.push_back(kGdn);
    else if (k == "csa") c.kinds.push_back(kCsa);
    else if (k == "hca") c.kinds.push_back(kHca);
    else throw std::runtime_error("unsupported block kind " + k);
    p = e + 1;
  }
  const bool any_attn = std::count(c.kinds.begin(), c.kinds.end(), kAttn) > 0;
  const bool any_gdn = c.has_gdn();
  if (cfg_int(kv, "physical_blocks", c.stem + static_cast<int>(c.kinds.size()) + c.tail, false) !=
      c.stem + static_cast<int>(c.kinds.size()) + c.tail)
    throw std::runtime_error("physical_blocks must equal stem + recurrent + tail blocks");
  c.attn_heads = cfg_int(kv, "attn.heads", 0, any_attn);
  c.attn_head_dim = cfg_int(kv, "attn.head_dim", 0, any_attn);
  c.window = cfg_int(kv, "attn.window", 0, any_attn);
  c.gdn_heads = cfg_int(kv, "gdn.qk_heads", 0, any_gdn);
  if (any_gdn && cfg_int(kv, "gdn.value_heads", c.gdn_heads, false) != c.gdn_heads)
    throw std::runtime_error("GDN q/k and value head counts must match");
  c.dk = cfg_int(kv, "gdn.qk_head_dim", 0, any_gdn);
  c.dv = cfg_int(kv, "gdn.value_head_dim", 0, any_gdn);
  c.conv_kernel = cfg_int(kv, "gdn.conv_kernel", 4, false);
  c.experts = cfg_int(kv, "moe.routed_experts", 0, true);
  c.top_k = cfg_int(kv, "moe.routed_top_k", 0, true);
  c.hidden = cfg_int(kv, "moe.expert_hidden", 0, true);
  c.shared = cfg_int(kv, "moe.shared_experts", 0, false);
  c.ctx = cfg_bool(kv, "router.context_aware", true);
  c.ctx_window = cfg_int(kv, "router.local_context", 128, false);
  c.latent = cfg_int(kv, "mla.latent_dim", 256, false);
  c.router_heads = cfg_int(kv, "router.query_heads", 4, false);
  c.router_head_dim = cfg_int(kv, "router.query_head_dim", 64, false);
  c.csa_ratio = cfg_int(kv, "csa.temporal_compression", 4, false);
  c.csa_window = cfg_int(kv, "csa.local_window", 128, false);
  c.csa_heads = cfg_int(kv, "csa.index_heads", 16, false);
  c.csa_head_dim = cfg_int(kv, "csa.index_head_dim", 128, false);
  c.csa_top_k = cfg_int(kv, "csa.index_top_k", 32, false);
  c.hca_ratio = cfg_int(kv, "hca.temporal_compression", 32, false);
  c.hca_window = cfg_int(kv, "hca.local_window", 128, false);
  c.hca_dense = cfg_bool(kv, "hca.dense_global_attention", true);
  c.hca_top_k = cfg_int(kv, "hca.global_top_k", 32, false);
  c.cmp_slots = cfg_int(kv, "memory.decode_slots", 256, false);
  auto eps = kv.find("rms_norm_eps");
  if (eps != kv.end()) c.eps = std::stof(eps->second);
  if (c.kinds.empty() || c.num_loops < 1 || c.vocab < 1 || c.d_model % 256 != 0 ||
      c.hidden < 2 || c.hidden % 2 != 0 || c.top_k < 1 || c.top_k > c.experts ||
      c.conv_kernel != 4 || c.shared < 0 || c.shared > 64 || c.stem < 0 || c.tail < 0 ||
      ((c.stem > 0 || c.tail > 0) && (c.dense_hidden < 2 || c.dense_hidden % 2 != 0)))
    throw std::runtime_error("unsupported model shape");
  if (c.ctx && (c.latent % 64 != 0 || c.latent > 512 || c.d_model > 1024 || c.ctx_window < 1))
    throw std::runtime_error("context-aware router needs mla.latent_dim % 64 == 0 and <= 512, "
                             "d_model <= 1024, router.local_context >= 1");
  if (c.ctx && std::count(c.kinds.begin(), c.kinds.end(), kHca) > 0) {
    if (c.router_heads < 1 || c.router_head_dim % 8 != 0 || c.hq() % 16 != 0)
      throw std::runtime_error("the router's latent attention needs router.query_heads * "
                               "router.query_head_dim % 16 == 0 and head_dim % 8 == 0");
    // both reference implementations build the router without this key
    // (model/model.py:112-117; llmy_cuda/src/config.cpp) and always attend to
    // the HCA summaries, so a file that turns it off asks for math neither runs
    if (!cfg_bool(kv, "router.use_hca_global_latents", true))
      throw std::runtime_error("router.use_hca_global_latents = 0 with HCA blocks: the "
                               "reference models ignore this key and always use the HCA "
                               "global branch");
  }
  if (c.mhc > 1 && (c.d_model > 4096 || c.mhc_iters < 0))
    throw std::runtime_error("mHC needs d_model <= 4096");
  // compressed-memory mixers: head widths the decode scoring splits over
  // lanes (16..256 or a multiple of 512), top-k <= 64, memory and window
  // within the kernels' LDS lists
  auto dh_ok = [](int d) {
    return d == 32 || d == 64 || d == 128 || d == 256 || (d % 512 == 0 && d <= 4096);
  };
  for (int kind : {kCsa, kHca}) {
    if (!c.has(kind)) continue;
    const CmpShape cs = c.cmp(kind);
    if (!dh_ok(cs.Dh) || cs.kw() % 16 != 0 || cs.W < 1 || cs.W > 4096 || cs.ratio < 1 ||
        cs.top_k < 0 || cs.top_k > 64 || c.cmp_slots < 1 || c.cmp_slots > 7168 || c.d_model > 8192)
      throw std::runtime_error("unsupported CSA / HCA shape");
  }
  return c;
}

float bf16_to_f32(uint16_t v) {
  uint32_t u = static_cast<uint32_t>(v) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

uint16_t f32_to_bf16(float f) {  // round to nearest even, NaN kept quiet
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

float f16_to_f32(uint16_t h) {
  const uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  float v;
  if (e == 0) v = std::ldexp(static_cast<float>(m), -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = std::ldexp(static_cast<float>(m | 0x400u), static_cast<int>(e) - 25);
  return s ? -v : v;
}

std::vector<float> as_f32(const TensorRef& t) {
  std::vector<float> out(static_cast<size_t>(t.numel()));
  for (size_t i = 0; i < out.size(); ++i) {
    if (t.dtype == 0) std::memcpy(&out[i], t.data + 4 * i, 4);
    else {
      uint16_t v;
      std::memcpy(&v, t.data + 2 * i, 2);
      out[i] = t.dtype == 2 ? bf16_to_f32(v) : f16_to_f32(v);
    }
  }
  return out;
}

std::vector<uint16_t> as_bf16(const TensorRef& t) {
  std::vector<uint16_t> out(static_cast<size_t>(t.numel()));
  if (t.dtype == 2) {
    std::memcpy(out.data(), t.data, out.size() * 2);
    return out;
  }
  const std::vector<float> f = as_f32(t);
  for (size_t i = 0; i < out.size(); ++i) out[i] = f32_to_bf16(f[i]);
  return out;
}

void expect_shape(const TensorRef& t, std::vector<int64_t> want, const std::string& name) {
  if (t.shape != want) throw std::runtime_error("unexpected shape for " + name);
}

struct Layer {
  int kind = kAttn;
  float* mix_norm = nullptr;
  float* ffn_norm = nullptr;
  float* router_norm = nullptr;
  float* w_router = nullptr;
  uint16_t* wqkv = nullptr;  // packed [3 H hd, D]
  uint16_t* wo = nullptr;    // packed [D, H hd]
  uint16_t* wproj = nullptr; // packed [N16, D]
  uint16_t* wout = nullptr;  // packed [D, H dv]
  float* bb = nullptr;
  float* conv = nullptr;     // [D, 4]
  float* decay = nullptr;
  uint16_t* w_gate_up = nullptr;  // packed per expert [E, 2H, D]
  uint16_t* w_down = nullptr;     // packed per expert [E, D, H]
  // context-aware router: latent encoder [L, D] + LayerNorm, gate (fp32);
  // local_context_out [D, L] and context_out [D, D] packed bf16
  float *ctx_down = nullptr, *ctx_ln_w = nullptr, *ctx_ln_b = nullptr, *ctx_gate = nullptr;
  uint16_t *ctx_local_out = nullptr, *ctx_out = nullptr;
  // mHC: the maps' projection theta (packed [n16, S D]) and fp32 parameters
  // (alpha = pre, post, residual)
  uint16_t* mhc_theta = nullptr;
  float *mhc_map_norm = nullptr, *mhc_pre_bias = nullptr, *mhc_post_bias = nullptr,
        *mhc_res_bias = nullptr, *mhc_alpha = nullptr, *mhc_gating = nullptr,
        *mhc_scale = nullptr, *mhc_ln_w = nullptr, *mhc_ln_b = nullptr;
  // CSA / HCA (packed bf16): query | key | value [2 Kw + D, D], the
  // compressor's key | value [Kw + D, D], [local_out | remote_out] [D, 2 D], out [D, D]
  uint16_t *cmp_wqkv = nullptr, *cmp_wc = nullptr, *cmp_wlr = nullptr, *cmp_wout = nullptr;
  // the context router's global branch (HCA blocks): hca_latent down [L, D]
  // (packed) + LayerNorm (fp32), latent attention q [HQ, D], k | v [2 HQ, L],
  // o [D, HQ] (packed)
  uint16_t *hca_lat_down = nullptr, *ctx_q = nullptr, *ctx_kv = nullptr, *ctx_o = nullptr;
  float *hca_lat_ln_w = nullptr, *hca_lat_ln_b = nullptr;
  // stem / tail blocks: the dense SwiGLU FFN as a one-expert stack (packed
  // gate | up [1, 2 Hd, D], down [1, D, Hd]) that the MoE kernels run with every
  // token routed to it at gate 1
  bool side = false;
  uint16_t *ffn_gate_up = nullptr, *ffn_down = nullptr;
};

struct Model {
  Config cfg;
  int loops = 0;  // loops a forward runs by default (llmy_set_num_loops)
  uint16_t* embed = nullptr;    // row-major [V, D] (token lookup)
  uint16_t* lm_head = nullptr;  // packed copy (tied LM head)
  float* final_norm = nullptr;
  float* stream_seed = nullptr;     // mHC: [S, D]
  uint16_t* mhc_collapse = nullptr; // mHC: packed [D, S D]
  std::vector<Layer> layers;        // the recurrent core
  std::vector<Layer> stem, tail;    // GDN + dense FFN blocks before / after the loops
  std::vector<void*> allocs;

  ~Model() {
    for (void* p : allocs) (void)hipFree(p);
  }
  template <typename T>
  T* alloc(size_t count) {
    void* p = nullptr;
    check_hip(hipMalloc(&p, std::max<size_t>(count, 1) * sizeof(T)), "hipMalloc (weights)");
    allocs.push_back(p);
    return static_cast<T*>(p);
  }
  template <typename T>
  T* upload(const std::vector<T>& host) {
    T* d = alloc<T>(host.size());
    check_hip(hipMemcpy(d, host.data(), host.size() * sizeof(T), hipMemcpyHostToDevice),
              "hipMemcpy (weights)");
    return d;
  }
  // [batch, N, K] row-major bf16 -> device, re-laid in the packed operand order.
  uint16_t* upload_packed(const std::vector<uint16_t>& host, int64_t batch, int N, int K) {
    void* tmp = nullptr;
    check_hip(hipMalloc(&tmp, host.size() * 2), "hipMalloc (staging)");
    std::unique_ptr<void, void (*)(void*)> guard(tmp, [](void* p) { (void)hipFree(p); });
    check_hip(hipMemcpy(tmp, host.data(), host.size() * 2, hipMemcpyHostToDevice), "hipMemcpy");
    uint16_t* out = alloc<uint16_t>(host.size());
    check_call(llmy_pack_weights_bf16(static_cast<const llmy_bf16*>(tmp), out, batch, N, K,
                                      nullptr),
               "llmy_pack_weights_bf16");
    check_hip(hipDeviceSynchronize(), "pack");
    return out;
  }
};

std::vector<uint16_t> concat_rows(std::initializer_list<std::vector<uint16_t>> parts, size_t pad_to) {
  std::vector<uint16_t> out;
  for (const auto& p : parts) out.insert(out.end(), p.begin(), p.end());
  out.resize(std::max(out.size(), pad_to), 0);
  return out;
}

// [N, K] -> [N, Kp] with zero columns K .. Kp-1: the weight of a GEMM whose
// input width is zero-padded to the kernels' multiple of 256 (its input goes
// through llmy_pad_cols_bf16).
std::vector<uint16_t> pad_cols(const std::vector<uint16_t>& w, int N, int K, int Kp) {
  if (K == Kp) return w;
  std::vector<uint16_t> out(static_cast<size_t>(N) * Kp, 0);
  for (int n = 0; n < N; ++n)
    std::memcpy(out.data() + static_cast<size_t>(n) * Kp, w.data() + static_cast<size_t>(n) * K,
                static_cast<size_t>(K) * 2);
  return out;
}

// Expert stacks with their hidden width H zero-padded to Hp: gate | up
// [EX, 2 Hp, D] (gate rows, zeros, up rows, zeros) and down [EX, D, Hp].
// Padded gate / up rows give activations silu(0) * 0 = 0 and padded down
// columns add nothing, so the result is the unpadded one.
void pad_hidden(std::vector<uint16_t>& gu, std::vector<uint16_t>& dn, int EX, int H, int Hp,
                int D) {
  if (H == Hp) return;
  std::vector<uint16_t> g2(static_cast<size_t>(EX) * 2 * Hp * D, 0);
  const size_t blk = static_cast<size_t>(H) * D, blkp = static_cast<size_t>(Hp) * D;
  for (int e = 0; e < EX; ++e) {
    std::memcpy(g2.data() + 2 * e * blkp, gu.data() + 2 * e * blk, blk * 2);
    std::memcpy(g2.data() + (2 * e + 1) * blkp, gu.data() + (2 * e + 1) * blk, blk * 2);
  }
  gu.swap(g2);
  dn = pad_cols(dn, EX * D, H, Hp);
}

std::unique_ptr<Model> load_model(const char* path) {
  Checkpoint ck;
  parse_checkpoint(path, ck);
  auto m = std::make_unique<Model>();
  Config& c = m->cfg;
  c = config_from(ck.config);
  m->loops = c.num_loops;
  const int D = c.d_model, V = c.vocab, E = c.experts, Hf = c.hidden;
  const auto& emb = ck.get("embed_tokens.weight");
  expect_shape(emb, {V, D}, "embed_tokens.weight");
  const std::vector<uint16_t> embed = as_bf16(emb);
  m->embed = m->upload(embed);
  m->lm_head = m->upload_packed(embed, 1, V, D);
  const auto& fn = ck.get("final_norm.weight");
  expect_shape(fn, {D}, "final_norm.weight");
  m->final_norm = m->upload(as_f32(fn));
  const int SM = c.mhc;
  if (SM > 1) {  // model.py:389-390,415-421 (stream_seed, mhc_collapse)
    const auto& sd = ck.get("stream_seed");
    expect_shape(sd, {SM, D}, "stream_seed");
    m->stream_seed = m->upload(as_f32(sd));
    const auto& cl = ck.get("mhc_collapse.weight");
    expect_shape(cl, {D, static_cast<int64_t>(SM) * D}, "mhc_collapse.weight");
    m->mhc_collapse = m->upload_packed(as_bf16(cl), 1, D, SM * D);
  }
  // One block under the name prefix p: a core block of `kind` (mixer + MoE), or
  // a stem / tail block (side: GDN mixer + dense FFN).
  auto load_block = [&](const std::string& p, int kind, bool side) {
    Layer L;
    L.kind = kind;
    L.side = side;
    auto vec_f32 = [&](const std::string& n, std::vector<int64_t> shape) {
      const auto& t = ck.get(p + n);
      expect_shape(t, shape, p + n);
      return m->upload(as_f32(t));
    };
    auto mat_bf16 = [&](const std::string& n, std::vector<int64_t> shape) {
      const auto& t = ck.get(p + n);
      expect_shape(t, shape, p + n);
      return as_bf16(t);
    };
    if (SM > 1) {  // the block's hyper-connection (mhc.py:63-84; names of model.cpp:34-63)
      auto scalar = [&](const std::string& n) {
        const auto& t = ck.get(p + n);
        if (!(t.shape.empty() || t.shape == std::vector<int64_t>{1}))
          throw std::runtime_error("unexpected shape for " + p + n);
        return as_f32(t)[0];
      };
      const int NT = 2 * SM + SM * SM;
      L.mhc_theta = m->upload_packed(
          concat_rows({mat_bf16("mhc.theta.weight", {NT, static_cast<int64_t>(SM) * D})},
                      static_cast<size_t>(c.mhc_n16()) * SM * D),
          1, c.mhc_n16(), SM * D);
      L.mhc_map_norm = vec_f32("mhc.mapping_norm.weight", {static_cast<int64_t>(SM) * D});
      L.mhc_pre_bias = vec_f32("mhc.pre_bias", {SM});
      L.mhc_post_bias = vec_f32("mhc.post_bias", {SM});
      L.mhc_res_bias = vec_f32("mhc.residual_bias", {SM, SM});
      L.mhc_alpha = m->upload(std::vector<float>{scalar("mhc.alpha_pre"), scalar("mhc.alpha_post"),
                                                 scalar("mhc.alpha_residual")});
      L.mhc_gating = m->upload(std::vector<float>{scalar("mhc.gating_logit")});
      L.mhc_scale = vec_f32("mhc.stream_scale", {SM, D});
      L.mhc_ln_w = vec_f32("mhc.stream_norm.weight", {D});
      L.mhc_ln_b = vec_f32("mhc.stream_norm.bias", {D});
    }
    L.mix_norm = vec_f32("mixer_norm.weight", {D});
    L.ffn_norm = vec_f32("ffn_norm.weight", {D});
    if (!side) {
      L.router_norm = vec_f32("moe.router.norm.weight", {D});
      L.w_router = vec_f32("moe.router.logits.weight", {E, D});
    }
    if (c.ctx && !side) {
      const int Lc = c.latent;
      L.ctx_down = vec_f32("moe.router.latent_memory.down.weight", {Lc, D});
      L.ctx_ln_w = vec_f32("moe.router.latent_memory.norm.weight", {Lc});
      L.ctx_ln_b = vec_f32("moe.router.latent_memory.norm.bias", {Lc});
      const auto& gt = ck.get(p + "moe.router.route_gate");  // a 0-d parameter
      if (!(gt.shape.empty() || gt.shape == std::vector<int64_t>{1}))
        throw std::runtime_error("unexpected shape for moe.router.route_gate");
      L.ctx_gate = m->upload(as_f32(gt));
      L.ctx_local_out = m->upload_packed(
          pad_cols(mat_bf16("moe.router.local_context_out.weight", {D, Lc}), D, Lc, c.latent_p()),
          1, D, c.latent_p());
      L.ctx_out = m->upload_packed(mat_bf16("moe.router.context_out.weight", {D, D}), 1, D, D);
      if (L.kind == kHca) {  // model.py:117, context_router.py:24 (model.cpp:98-104,234)
        const int HQ = c.hq();
        L.hca_lat_down = m->upload_packed(mat_bf16("hca_latent.down.weight", {Lc, D}), 1, Lc, D);
        L.hca_lat_ln_w = vec_f32("hca_latent.norm.weight", {Lc});
        L.hca_lat_ln_b = vec_f32("hca_latent.norm.bias", {Lc});
        L.ctx_q = m->upload_packed(mat_bf16("moe.router.latent_attention.q.weight", {HQ, D}), 1,
                                   HQ, D);
        L.ctx_kv = m->upload_packed(
            pad_cols(concat_rows({mat_bf16("moe.router.latent_attention.k.weight", {HQ, Lc}),
                                  mat_bf16("moe.router.latent_attention.v.weight", {HQ, Lc})}, 0),
                     2 * HQ, Lc, c.latent_p()),
            1, 2 * HQ, c.latent_p());
        L.ctx_o = m->upload_packed(
            pad_cols(mat_bf16("moe.router.latent_attention.o.weight", {D, HQ}), D, HQ, c.hq_p()),
            1, D, c.hq_p());
      }
    }
    if (L.kind == kCsa || L.kind == kHca) {
      // model/layers/csa.py:21-29, hca.py:24-30 (names of llmy_cuda/src/model.cpp:139-160)
      const int Kw = c.cmp(L.kind).kw();
      L.cmp_wqkv = m->upload_packed(concat_rows({mat_bf16("mixer.query.weight", {Kw, D}),
                                                 mat_bf16("mixer.key.weight", {Kw, D}),
                                                 mat_bf16("mixer.value.weight", {D, D})}, 0),
                                    1, 2 * Kw + D, D);
      L.cmp_wc = m->upload_packed(concat_rows({mat_bf16("mixer.compressor.key.weight", {Kw, D}),
                                               mat_bf16("mixer.compressor.value.weight", {D, D})},
                                              0),
                                  1, Kw + D, D);
      const auto lo = mat_bf16("mixer.local_out.weight", {D, D});
      const auto ro = mat_bf16(L.kind == kCsa ? "mixer.remote_out.weight" : "mixer.global_out.weight",
                               {D, D});
      std::vector<uint16_t> lr(static_cast<size_t>(D) * 2 * D);
      for (int i = 0; i < D; ++i) {  // row i: local_out[i, :] then remote_out[i, :]
        std::memcpy(lr.data() + static_cast<size_t>(i) * 2 * D, lo.data() + static_cast<size_t>(i) * D,
                    static_cast<size_t>(D) * 2);
        std::memcpy(lr.data() + static_cast<size_t>(i) * 2 * D + D,
                    ro.data() + static_cast<size_t>(i) * D, static_cast<size_t>(D) * 2);
      }
      L.cmp_wlr = m->upload_packed(lr, 1, D, 2 * D);
      L.cmp_wout = m->upload_packed(mat_bf16("mixer.out.weight", {D, D}), 1, D, D);
    } else if (L.kind == kAttn) {
      const int W = c.attn_heads * c.attn_head_dim;
      if (W % 16 != 0 || W % 256 != 0 || (c.attn_head_dim != 64 && c.attn_head_dim != 128))
        throw std::runtime_error("unsupported attention shape");
      const auto wqkv = concat_rows({mat_bf16("mixer.q.weight", {W, D}),
                                     mat_bf16("mixer.k.weight", {W, D}),
                                     mat_bf16("mixer.v.weight", {W, D})}, 0);
      L.wqkv = m->upload_packed(wqkv, 1, 3 * W, D);
      L.wo = m->upload_packed(mat_bf16("mixer.o.weight", {D, W}), 1, D, W);
    } else {
      const int H = c.gdn_heads, HK = H * c.dk, HV = H * c.dv;
      if (HV % 256 != 0 || (c.dk != 64 && c.dk != 128) || c.dk != c.dv)
        throw std::runtime_error("unsupported GDN shape");
      const auto wproj = concat_rows({mat_bf16("mixer.q_proj.weight", {HK, D}),
                                      mat_bf16("mixer.k_proj.weight", {HK, D}),
                                      mat_bf16("mixer.v_proj.weight", {HV, D}),
                                      mat_bf16("mixer.gate_proj.weight", {HV, D}),
                                      mat_bf16("mixer.beta_proj.weight", {H, D})},
                                     static_cast<size_t>(c.nproj16()) * D);
      L.wproj = m->upload_packed(wproj, 1, c.nproj16(), D);
      L.wout = m->upload_packed(mat_bf16("mixer.out_proj.weight", {D, HV}), 1, D, HV);
      L.bb = vec_f32("mixer.beta_proj.bias", {H});
      L.decay = vec_f32("mixer.decay_logit", {H});
      const auto& cv = ck.get(p + "mixer.conv.weight");
      if (cv.shape != std::vector<int64_t>{D, 1, 4} && cv.shape != std::vector<int64_t>{D, 4})
        throw std::runtime_error("unexpected conv shape");
      L.conv = m->upload(as_f32(cv));
    }
    if (side) {
      // the dense SwiGLU FFN (dense_ffn.py:9-11; names of llmy_cuda/src/model.cpp:81-87)
      const int Hd = c.dense_hidden;
      auto gu = concat_rows({mat_bf16("ffn.gate_proj.weight", {Hd, D}),
                             mat_bf16("ffn.up_proj.weight", {Hd, D})}, 0);
      auto dn = mat_bf16("ffn.down_proj.weight", {D, Hd});
      pad_hidden(gu, dn, 1, Hd, c.dense_p(), D);
      L.ffn_gate_up = m->upload_packed(gu, 1, 2 * c.dense_p(), D);
      L.ffn_down = m->upload_packed(dn, 1, D, c.dense_p());
      return L;
    }
    // Routed experts, then the S shared experts (moe.shared.*, stacked
    // [S, H, D] / [S, D, H] by the converter) as experts E .. E+S-1.
    const int S = c.shared, EX = E + S;
    const auto g = mat_bf16("moe.experts.gate_proj.weight", {E, Hf, D});
    const auto u = mat_bf16("moe.experts.up_proj.weight", {E, Hf, D});
    auto dn = mat_bf16("moe.experts.down_proj.weight", {E, D, Hf});
    std::vector<uint16_t> sg, su;
    if (S > 0) {
      sg = mat_bf16("moe.shared.gate_proj.weight", {S, Hf, D});
      su = mat_bf16("moe.shared.up_proj.weight", {S, Hf, D});
      const auto sd = mat_bf16("moe.shared.down_proj.weight", {S, D, Hf});
      dn.insert(dn.end(), sd.begin(), sd.end());
    }
    std::vector<uint16_t> gu(static_cast<size_t>(EX) * 2 * Hf * D);
    const size_t blk = static_cast<size_t>(Hf) * D;
    for (int e = 0; e < EX; ++e) {  // [E+S, 2H, D]: gate rows, then up rows
      const uint16_t* ge = e < E ? g.data() + e * blk : sg.data() + (e - E) * blk;
      const uint16_t* ue = e < E ? u.data() + e * blk : su.data() + (e - E) * blk;
      std::memcpy(gu.data() + 2 * e * blk, ge, blk * 2);
      std::memcpy(gu.data() + (2 * e + 1) * blk, ue, blk * 2);
    }
    pad_hidden(gu, dn, EX, Hf, c.hidden_p(), D);
    L.w_gate_up = m->upload_packed(gu, EX, 2 * c.hidden_p(), D);
    L.w_down = m->upload_packed(dn, EX, D, c.hidden_p());
    return L;
  };
  for (int i = 0; i < c.stem; ++i)
    m->stem.push_back(load_block("stem." + std::to_string(i) + ".", kGdn, true));
  for (size_t l = 0; l < c.kinds.size(); ++l)
    m->layers.push_back(load_block("recurrent_core." + std::to_string(l) + ".", c.kinds[l], false));
  for (int i = 0; i < c.tail; ++i)
    m->tail.push_back(load_block("tail." + std::to_string(i) + ".", kGdn, true));
  return m;
}

// ------------------------------------------------------------------ state
struct DeviceArena {
  std::vector<void*> ptrs;
  ~DeviceArena() { release(); }
  void release() {
    for (void* p : ptrs) (void)hipFree(p);
    ptrs.clear();
  }
  template <typename T>
  T* zeros(size_t count) {
    void* p = nullptr;
    const size_t bytes = std::max<size_t>(count, 1) * sizeof(T);
    check_hip(hipMalloc(&p, bytes), "hipMalloc (state)");
    ptrs.push_back(p);
    check_hip(hipMemset(p, 0, bytes), "hipMemset (state)");
    return static_cast<T*>(p);
  }
};

struct LayerState {
  uint16_t* k = nullptr;  // [B, H, W, hd]
  uint16_t* v = nullptr;
  float* S = nullptr;       // [B, H, dk, dv]
  uint16_t* hist = nullptr; // [B, 3, D]
  float* ring = nullptr;    // context router: [B, W, L], the last W latents (slot pos % W)
  size_t k_bytes = 0, s_bytes = 0, hist_bytes = 0, ring_bytes = 0;
  // CSA / HCA: local ring keys [B, W, Kw] / values [B, W, D], memory slots keys
  // [B, C, Kw] / values [B, C, D] / tags [B, C] (position + 1, 0 empty), summaries
  // emitted per row [B], the incomplete block's sum [B, D] fp32 and count [B]
  uint16_t *lk = nullptr, *lv = nullptr, *mk = nullptr, *mv = nullptr;
  int32_t *mtag = nullptr, *mcount = nullptr, *pcnt = nullptr;
  float* psum = nullptr;
  // HCA with the context router: the router's keys / values [B, C, HQ] of each
  // summary's latent, their tags and count (kept as the memory's)
  uint16_t *rk = nullptr, *rv = nullptr;
  int32_t *rtag = nullptr, *rcount = nullptr;
  std::vector<std::pair<void*, size_t>> cmp_bufs;  // every CSA / HCA buffer and its bytes
};

struct Buffers {  // activations for `rows` token rows
  int rows = 0;
  float *x = nullptr, *proj = nullptr, *cg = nullptr, *gates = nullptr, *y = nullptr;
  float *beta = nullptr, *g = nullptr;
  float* parts = nullptr;  // decode: mixer output projection partials [n, rows, D]
  int max_parts = 0;
  float* proj_parts = nullptr;  // decode: GDN input projection partials [D/256, rows, nproj16]
  float* qkv_parts = nullptr;   // decode: attention q/k/v projection partials [D/256, rows, 3 Hhd]
  uint16_t *h = nullptr, *qkv = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *ao = nullptr,
           *go = nullptr, *act = nullptr, *gq = nullptr, *gk = nullptr, *gv = nullptr;
  int32_t *tokens = nullptr, *idx = nullptr, *counts = nullptr, *offsets = nullptr,
          *sorted = nullptr, *route_pos = nullptr;
  int32_t* idx_all = nullptr;  // shared experts: [rows, k + S] routes
  float* gates_all = nullptr;
  // context router: local [rows, D], lat [rows, L], c [rows, D], logits [rows, E] fp32;
  // window means [rows, L] and local_context_out [rows, D] bf16
  float *c_local = nullptr, *c_lat = nullptr, *c_c = nullptr, *c_logits = nullptr;
  uint16_t *c_ctx = nullptr, *c_d = nullptr;
  // zero-padded GEMM inputs (latent_dim / query width not a multiple of 256):
  // window means [rows, Lp], summary latents [rows, Lp], latent attention [rows, HQp]
  uint16_t *c_ctx_p = nullptr, *g_lat_p = nullptr, *g_att_p = nullptr;
  // stem / tail dense FFN: activation [rows, Hdp], one route per row (expert 0,
  // gate 1)
  uint16_t* dact = nullptr;
  int32_t* dids = nullptr;
  float* dgates = nullptr;
  // the global branch (HCA): summary values [rows, D] / latents [rows, L] fp32 and
  // bf16 / router k | v [rows, 2 HQ]; local in bf16, q and attention [rows, HQ],
  // local_context_out + o in fp32 [rows, D]
  uint16_t *g_val = nullptr, *g_lat = nullptr, *g_kvr = nullptr, *g_lq = nullptr,
           *g_q = nullptr, *g_att = nullptr;
  float *g_lat_raw = nullptr, *g_t = nullptr;
  // mHC: streams X [rows, S, D], their bf16 copy [rows, S D] (GEMM operand),
  // map logits [rows, n16], maps [rows, S + S^2], a sublayer's output U
  // [rows, D]; all-ones row mask (clearing U) and identity route positions
  float *mX = nullptr, *mraw = nullptr, *mmaps = nullptr, *mU = nullptr;
  uint16_t* mxb = nullptr;
  int32_t *mones = nullptr, *mident = nullptr;
  // CSA / HCA: projection [rows, 2 Kw + D], branch outputs [rows, 2 D], their
  // projection [rows, D], the compressor's mean [rows, D] and emit flags
  // (decode), block means [B T/ratio, D] (prefill), summaries [., Kw + D], lists
  uint16_t *cqkv = nullptr, *cloc = nullptr, *cy = nullptr, *cmean = nullptr, *ckv = nullptr;
  int32_t* cemit = nullptr;
  void* cws = nullptr;
  int64_t cws_bytes = 0;
  void* ws = nullptr;
  int64_t ws_bytes = 0;
  DeviceArena arena;
};

struct State {
  Model* model = nullptr;
  int B = 1;
  int last_loops = 0;
  hipStream_t stream = nullptr;         // every launch of this state (default priority)
  std::map<int, hipGraphExec_t> graphs; // decode step per loop count, captured on first use
  std::vector<int32_t> hpos;            // host copy of pos
  std::vector<LayerState> layers;  // index loop * n_layers + layer
  std::vector<LayerState> side;    // stem blocks, then tail blocks (GDN state each)
  DeviceArena arena;
  int32_t* pos = nullptr;    // [B] device: absolute position of the next token
  int32_t* reset_mask = nullptr;  // [B] device: rows of the last llmy_state_reset_rows
  float* logits = nullptr;   // [B, V]
  int32_t* next = nullptr;   // [B]
  Buffers step;              // decode: B rows
  std::unique_ptr<Buffers> seq;  // prefill: B*T rows, grown on demand

  ~State() {
    if (stream) (void)hipStreamSynchronize(stream);
    for (auto& kv : graphs) (void)hipGraphExecDestroy(kv.second);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

void alloc_buffers(const Config& c, int rows, int B, int T, Buffers& b) {
  const int D = c.d_model, k = c.top_k, kx = c.routes(), EX = c.all_experts();
  b.rows = rows;
  b.x = b.arena.zeros<float>(static_cast<size_t>(rows) * D);
  b.h = b.arena.zeros<uint16_t>(static_cast<size_t>(rows) * D);
  const int Hhd = c.attn_heads * c.attn_head_dim;
  b.qkv = b.arena.zeros<uint16_t>(static_cast<size_t>(rows) * 3 * std::max(Hhd, 1));
  b.q = b.qkv;
  b.k = b.qkv + static_cast<size_t>(rows) * std::max(Hhd, 1);
  b.v = b.qkv + 2 * static_cast<size_t>(rows) * std::max(Hhd, 1);
  b.ao = b.arena.zeros<uint16_t>(static_cast<size_t>(rows) * std::max(Hhd, 1));
  const int HK = c.gdn_heads * c.dk, HV = c.gdn_heads * c.dv;
  b.proj = b.arena.zeros<float>(static_cast<size_t>(rows) * c.nproj16());
  b.go = b.arena.zeros<uint16_t>(static_cast<size_t>(rows) * std::max(HV, 1));
  b.cg = b.arena.zeros<float>(static_cast<size_t>(rows) * D);
  b.gq = b.arena.zeros<uint16_t>(static_cast<size_t>(rows) * std::max(HK, 1));
  b.gk = b.arena.zeros<uint16_t>(static_cast<size_t>(rows) * std::max(HK, 1));
  b.gv = b.arena.zeros<uint16_t>(static_cast<size_t>(rows) * std::max(HV, 1));
  b.beta = b.arena.zeros<float>(static_cast<size_t>(rows) * std::max(c.gdn_heads, 1));
  b.g = b.arena.zeros<float>(static_cast<size_t>(rows) * std::max(c.gdn_heads, 1));
  b.tokens = b.arena.zeros<int32_t>(rows);
  b.idx = b.arena.zeros<int32_t>(static_cast<size_t>(rows) * k);
  b.gates = b.arena.zeros<float>(static_cast<size_t>(rows) * k);
  if (c.shared > 0) {  // the router's routes plus the always-on shared ones
    b.idx_all = b.arena.zeros<int32_t>(static_cast<size_t>(rows) * kx);
    b.gates_all = b.arena.zeros<float>(static_cast<size_t>(rows) * kx);
  }
  if (c.ctx) {
    b.c_local = b.arena.zeros<float>(static_cast<size_t>(rows) * D);
    b.c_lat = b.arena.zeros<float>(static_cast<size_t>(rows) * c.latent);
    b.c_c = b.arena.zeros<float>(static_cast<size_t>(rows) * D);
    b.c_logits = b.arena.zeros<float>(static_cast<size_t>(rows) * c.experts);
    b.c_ctx = b.arena.zeros<uint16_t>(static_cast<size_t>(rows) * c.latent);
    b.c_ctx_p = b.arena.zeros<uint16_t>(static_cast<size_t>(rows) * c.latent_p());
    b.c_d = b.arena.zeros<uint16_t>(static_cast<size_t>(rows) * D);
    if (c.has(kHca)) {
      const size_t R = rows, HQ = c.hq(), Lc = c.latent;
      b.g_val = b.arena.zeros<uint16_t>(R * D);
      b.g_lat_raw = b.arena.zeros<float>(R * Lc);
      b.g_lat = b.arena.zeros<uint16_t>(R * Lc);
      b.g_lat_p = b.arena.zeros<uint16_t>(R * c.latent_p());
      b.g_att_p = b.arena.zeros<uint16_t>(R * c.hq_p());
      b.g_kvr = b.arena.zeros<uint16_t>(R * 2 * HQ);
      b.g_lq = b.arena.zeros<uint16_t>(R * D);
      b.g_q = b.arena.zeros<uint16_t>(R * HQ);
      b.g_att = b.arena.zeros<uint16_t>(R * HQ);
      b.g_t = b.arena.zeros<float>(R * D);
    }
  }
  if (c.mhc > 1) {
    const size_t S = c.mhc;
    b.mX = b.arena.zeros<float>(static_cast<size_t>(rows) * S * D);
    b.mxb = b.arena.zeros<uint16_t>(static_cast<size_t>(rows) * S * D);
    b.mraw = b.arena.zeros<float>(static_cast<size_t>(rows) * c.mhc_n16());
    b.mmaps = b.arena.zeros<float>(static_cast<size_t>(rows) * (S + S * S));
    b.mU = b.arena.zeros<float>(static_cast<size_t>(rows) * D);
    std::vector<int32_t> ones(rows, 1), ident(static_cast<size_t>(rows) * kx);
    for (size_t i = 0; i < ident.size(); ++i) ident[i] = static_cast<int32_t>(i);
    b.mones = b.arena.zeros<int32_t>(rows);
    b.mident = b.arena.zeros<int32_t>(ident.size());
    check_hip(hipMemcpy(b.mones, ones.data(), ones.size() * 4, hipMemcpyHostToDevice), "ones");
    check_hip(hipMemcpy(b.mident, ident.data(), ident.size() * 4, hipMemcpyHostToDevice),
              "ident");
  }
  b.counts = b.arena.zeros<int32_t>(EX);
  b.offsets = b.arena.zeros<int32_t>(EX + 1);
  b.sorted = b.arena.zeros<int32_t>(static_cast<size_t>(rows) * kx);
  b.route_pos = b.arena.zeros<int32_t>(static_cast<size_t>(rows) * kx);
  b.act = b.arena.zeros<uint16_t>(static_cast<size_t>(rows) * kx * c.hidden_p());
  if (c.stem > 0 || c.tail > 0) {
    b.dact = b.arena.zeros<uint16_t>(static_cast<size_t>(rows) * c.dense_p());
    b.dids = b.arena.zeros<int32_t>(rows);
    b.dgates = b.arena.zeros<float>(rows);
    const std::vector<float> ones(rows, 1.0f);
    check_hip(hipMemcpy(b.dgates, ones.data(), ones.size() * 4, hipMemcpyHostToDevice), "ones");
  }
  b.y = b.arena.zeros<float>(static_cast<size_t>(rows) * kx * D);
  if (T == 1 && rows <= 64 && Hhd % 256 == 0 && HV % 256 == 0 &&
      std::max(Hhd, HV) / 256 <= 8) {
    b.max_parts = std::max(Hhd, HV) / 256;
    b.parts = b.arena.zeros<float>(static_cast<size_t>(b.max_parts) * rows * D);
  }
  if (T == 1 && rows <= 64 && D % 256 == 0 && D / 256 <= 8 && c.has_gdn())
    b.proj_parts = b.arena.zeros<float>(static_cast<size_t>(D / 256) * rows * c.nproj16());
  if (T == 1 && rows <= 64 && D % 256 == 0 && D / 256 <= 8 && c.has(kAttn))
    b.qkv_parts = b.arena.zeros<float>(static_cast<size_t>(D / 256) * rows * 3 * Hhd);
  if (c.has(kCsa) || c.has(kHca)) {
    int kw = 0, rmin = 1 << 30;
    int64_t ws = 16;
    for (int kind : {kCsa, kHca}) {
      if (!c.has(kind)) continue;
      const CmpShape cs = c.cmp(kind);
      kw = std::max(kw, cs.kw());
      rmin = std::min(rmin, cs.ratio);
      const int slots = T == 1 ? c.cmp_slots : std::max(T / cs.ratio, 1);
      const int dec = T == 1 ? 1 : 0;
      ws = std::max({ws, llmy_cmp_workspace_bytes(rows, cs.H, cs.W, 0, dec),
                     llmy_cmp_workspace_bytes(rows, cs.H, slots, cs.top_k, dec)});
    }
    if (ws < 0) throw std::runtime_error("CSA / HCA workspace size");
    const size_t nsum = T == 1 ? static_cast<size_t>(rows) : static_cast<size_t>(B) * (T / rmin);
    b.cqkv = b.arena.zeros<uint16_t>(static_cast<size_t>(rows) * (2 * kw + D));
    b.cloc = b.arena.zeros<uint16_t>(static_cast<size_t>(rows) * 2 * D);
    b.cy = b.arena.zeros<uint16_t>(static_cast<size_t>(rows) * D);
    b.cmean = b.arena.zeros<uint16_t>(std::max(nsum, static_cast<size_t>(1)) * D);
    b.ckv = b.arena.zeros<uint16_t>(std::max(nsum, static_cast<size_t>(1)) * (kw + D));
    b.cemit = b.arena.zeros<int32_t>(rows);
    b.cws_bytes = ws;
    b.cws = b.arena.zeros<unsigned char>(static_cast<size_t>(ws));
  }
  if (T > 1 && c.has_gdn()) {
    b.ws_bytes = llmy_gdn_prefill_workspace_bytes(B, T, c.gdn_heads, c.dk, c.dv);
    if (b.ws_bytes < 0) throw std::runtime_error("GDN prefill workspace size");
    b.ws = b.arena.zeros<unsigned char>(static_cast<size_t>(b.ws_bytes));
  }
}

std::unique_ptr<State> new_state(Model* m, int B) {
  if (B < 1) throw std::runtime_error("batch must be >= 1");
  const Config& c = m->cfg;
  auto s = std::make_unique<State>();
  s->model = m;
  s->B = B;
  const int D = c.d_model;
  for (int loop = 0; loop < c.num_loops; ++loop) {
    for (int kind : c.kinds) {
      LayerState L;
      if (kind == kCsa || kind == kHca) {
        const CmpShape cs = c.cmp(kind);
        const size_t Bz = B, W = cs.W, C = c.cmp_slots, Kw = cs.kw(), Dz = D;
        auto add = [&](auto* p, size_t bytes) {
          L.cmp_bufs.emplace_back(static_cast<void*>(p), bytes);
          return p;
        };
        L.lk = add(s->arena.zeros<uint16_t>(Bz * W * Kw), Bz * W * Kw * 2);
        L.lv = add(s->arena.zeros<uint16_t>(Bz * W * Dz), Bz * W * Dz * 2);
        L.mk = add(s->arena.zeros<uint16_t>(Bz * C * Kw), Bz * C * Kw * 2);
        L.mv = add(s->arena.zeros<uint16_t>(Bz * C * Dz), Bz * C * Dz * 2);
        L.mtag = add(s->arena.zeros<int32_t>(Bz * C), Bz * C * 4);
        L.mcount = add(s->arena.zeros<int32_t>(Bz), Bz * 4);
        L.psum = add(s->arena.zeros<float>(Bz * Dz), Bz * Dz * 4);
        L.pcnt = add(s->arena.zeros<int32_t>(Bz), Bz * 4);
        if (kind == kHca && c.ctx) {
          const size_t HQ = c.hq();
          L.rk = add(s->arena.zeros<uint16_t>(Bz * C * HQ), Bz * C * HQ * 2);
          L.rv = add(s->arena.zeros<uint16_t>(Bz * C * HQ), Bz * C * HQ * 2);
          L.rtag = add(s->arena.zeros<int32_t>(Bz * C), Bz * C * 4);
          L.rcount = add(s->arena.zeros<int32_t>(Bz), Bz * 4);
        }
      } else if (kind == kAttn) {
        const size_t n = static_cast<size_t>(B) * c.attn_heads * c.window * c.attn_head_dim;
        L.k = s->arena.zeros<uint16_t>(n);
        L.v = s->arena.zeros<uint16_t>(n);
        L.k_bytes = n * 2;
      } else {
        const size_t n = static_cast<size_t>(B) * c.gdn_heads * c.dk * c.dv;
        L.S = s->arena.zeros<float>(n);
        L.s_bytes = n * 4;
        L.hist = s->arena.zeros<uint16_t>(static_cast<size_t>(B) * 3 * D);
        L.hist_bytes = static_cast<size_t>(B) * 3 * D * 2;
      }
      if (c.ctx) {
        const size_t n = static_cast<size_t>(B) * c.ctx_window * c.latent;
        L.ring = s->arena.zeros<float>(n);
        L.ring_bytes = n * 4;
      }
      s->layers.push_back(L);
    }
  }
  for (int i = 0; i < c.stem + c.tail; ++i) {  // stem / tail GDN states
    LayerState L;
    const size_t n = static_cast<size_t>(B) * c.gdn_heads * c.dk * c.dv;
    L.S = s->arena.zeros<float>(n);
    L.s_bytes = n * 4;
    L.hist = s->arena.zeros<uint16_t>(static_cast<size_t>(B) * 3 * D);
    L.hist_bytes = static_cast<size_t>(B) * 3 * D * 2;
    s->side.push_back(L);
  }
  check_hip(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking), "hipStreamCreate");
  s->hpos.assign(B, 0);
  s->pos = s->arena.zeros<int32_t>(B);
  s->reset_mask = s->arena.zeros<int32_t>(B);
  s->logits = s->arena.zeros<float>(static_cast<size_t>(B) * c.vocab);
  s->next = s->arena.zeros<int32_t>(B);
  alloc_buffers(c, B, B, 1, s->step);
  return s;
}

void reset_state(State& s) {
  std::vector<LayerState*> all;
  for (auto& L : s.layers) all.push_back(&L);
  for (auto& L : s.side) all.push_back(&L);
  for (LayerState* Lp : all) {
    LayerState& L = *Lp;
    if (L.k) {
      check_hip(hipMemsetAsync(L.k, 0, L.k_bytes, s.stream), "reset");
      check_hip(hipMemsetAsync(L.v, 0, L.k_bytes, s.stream), "reset");
    }
    if (L.S) {
      check_hip(hipMemsetAsync(L.S, 0, L.s_bytes, s.stream), "reset");
      check_hip(hipMemsetAsync(L.hist, 0, L.hist_bytes, s.stream), "reset");
    }
    if (L.ring) check_hip(hipMemsetAsync(L.ring, 0, L.ring_bytes, s.stream), "reset");
    for (auto& pb : L.cmp_bufs) check_hip(hipMemsetAsync(pb.first, 0, pb.second, s.stream), "reset");
  }
  check_hip(hipMemsetAsync(s.pos, 0, sizeof(int32_t) * s.B, s.stream), "reset");
  check_hip(hipStreamSynchronize(s.stream), "reset");
  s.hpos.assign(s.B, 0);
  s.last_loops = 0;
}

// Rows b with mask[b] != 0 (host or device int32 [B]) start over: every
// per-row state buffer is zeroed by a kernel (no memory set) and the next
// position is 0 (recurrent_state.py:213-225, model.py:814-822).
void reset_rows(State& s, const int32_t* mask) {
  check_hip(hipMemcpyAsync(s.reset_mask, mask, sizeof(int32_t) * s.B, hipMemcpyDefault, s.stream),
            "reset mask");
  auto zero = [&](void* p, size_t bytes) {
    if (p)
      check_call(llmy_zero_rows(p, static_cast<int64_t>(bytes / s.B), s.B, s.reset_mask, s.stream),
                 "llmy_zero_rows");
  };
  std::vector<LayerState*> all;
  for (auto& L : s.layers) all.push_back(&L);
  for (auto& L : s.side) all.push_back(&L);
  for (LayerState* Lp : all) {
    LayerState& L = *Lp;
    zero(L.k, L.k_bytes);
    zero(L.v, L.k_bytes);
    zero(L.S, L.s_bytes);
    zero(L.hist, L.hist_bytes);
    zero(L.ring, L.ring_bytes);
    for (auto& pb : L.cmp_bufs) zero(pb.first, pb.second);
  }
  zero(s.pos, sizeof(int32_t) * s.B);
  std::vector<int32_t> host(s.B);
  check_hip(hipMemcpyAsync(host.data(), s.reset_mask, sizeof(int32_t) * s.B, hipMemcpyDeviceToHost,
                           s.stream),
            "reset mask");
  check_hip(hipStreamSynchronize(s.stream), "reset rows");
  for (int b = 0; b < s.B; ++b)
    if (host[b] != 0) s.hpos[b] = 0;
}

// ------------------------------------------------------------------ forward
constexpr int kStoreBf16 = 0, kStoreF32 = 1, kResidAdd = 2, kResidGated = 3, kPartialF32 = 4,
              kPacked = 1;

void linear(const uint16_t* x, const uint16_t* w, void* out, const float* aux, int M, int N, int K,
            int epi, hipStream_t st) {
  check_call(llmy_linear_bf16(x, w, out, aux, M, N, K, epi, kPacked, st), "llmy_linear_bf16");
}

// Decode sizes for which the MoE front end is the fused router
// (llmy_moe_route_decode) with route-indexed experts.
// The fused norm + router kernel (llmy_moe_route_decode) takes any number of
// rows at these sizes; the route-indexed decode experts also need few routes.
bool router_fusable(const Config& c) {
  const int D = c.d_model;
  return static_cast<long long>(c.experts) * D <= 24576 && (D == 256 || D == 512 || D == 1024) &&
         c.top_k <= 8;
}

bool fused_route(const Config& c, int rows) { return router_fusable(c) && rows * c.routes() <= 2048; }

// The context-aware routing of b.h (llmy_router_context_*): the ids and gates
// into b.idx / b.gates.  Rows are nseq sequences of rows / nseq tokens at
// positions pos[b] + t (pos NULL: a prompt from 0); `ring` is the block's
// latent window state.  On an HCA block with the router's summary memory
// (ls->rk) the global branch's latent attention is added to
// local_context_out(ctx).  GEMM inputs narrower than their padded weights go
// through llmy_pad_cols_bf16.  The kernels and their order are the Python
// engine's (ops.router_context).
void context_route(const Model& m, const Layer& L, Buffers& b, int rows, float* ring,
                   const int32_t* pos, int nseq, const LayerState* ls, hipStream_t st) {
  const Config& c = m.cfg;
  const int D = c.d_model, E = c.experts, k = c.top_k, Lc = c.latent, Lp = c.latent_p();
  check_call(llmy_router_context_latent_f32(b.h, L.router_norm, L.ctx_down, L.ctx_ln_w,
                                            L.ctx_ln_b, b.c_local, b.c_lat, rows, D, Lc, c.eps,
                                            1e-5f, st),
             "llmy_router_context_latent_f32");
  check_call(llmy_router_context_window(b.c_lat, ring, pos, b.c_ctx, nseq, rows / nseq,
                                        c.ctx_window, Lc, st),
             "llmy_router_context_window");
  const uint16_t* ctx = b.c_ctx;
  if (Lp != Lc) {
    check_call(llmy_pad_cols_bf16(b.c_ctx, b.c_ctx_p, rows, Lc, Lp, st), "llmy_pad_cols_bf16");
    ctx = b.c_ctx_p;
  }
  if (ls && ls->rk) {
    // the global branch: local_context_out(ctx) + o(latent attention of
    // q(local) over the block's summaries), rounded once to bf16
    const int HQ = c.hq(), HQp = c.hq_p();
    linear(ctx, L.ctx_local_out, b.g_t, nullptr, rows, D, Lp, kStoreF32, st);
    check_call(llmy_f32_to_bf16(b.c_local, b.g_lq, static_cast<int64_t>(rows) * D, st),
               "llmy_f32_to_bf16");
    linear(b.g_lq, L.ctx_q, b.g_q, nullptr, rows, HQ, D, kStoreBf16, st);
    check_call(llmy_latent_attn_bf16(b.g_q, HQ, ls->rk, ls->rv, ls->rtag, pos, b.g_att, HQ, nseq,
                                     rows / nseq, c.cmp_slots, c.router_heads, c.router_head_dim,
                                     1.0f / std::sqrt(static_cast<float>(c.router_head_dim)), st),
               "llmy_latent_attn_bf16");
    const uint16_t* att = b.g_att;
    if (HQp != HQ) {
      check_call(llmy_pad_cols_bf16(b.g_att, b.g_att_p, rows, HQ, HQp, st), "llmy_pad_cols_bf16");
      att = b.g_att_p;
    }
    linear(att, L.ctx_o, b.g_t, nullptr, rows, D, HQp, kResidAdd, st);
    check_call(llmy_f32_to_bf16(b.g_t, b.c_d, static_cast<int64_t>(rows) * D, st),
               "llmy_f32_to_bf16");
  } else {
    linear(ctx, L.ctx_local_out, b.c_d, nullptr, rows, D, Lp, kStoreBf16, st);
  }
  linear(b.c_d, L.ctx_out, b.c_c, nullptr, rows, D, D, kStoreF32, st);
  check_call(llmy_router_context_logits_f32(b.c_local, b.c_c, L.ctx_gate, L.w_router, b.c_logits,
                                            rows, D, E, st),
             "llmy_router_context_logits_f32");
  check_call(llmy_router_topk_logits_f32(b.c_logits, b.idx, b.gates, rows, E, k, st),
             "llmy_router_topk_logits_f32");
}

// MoE of core block L over `rows` rows (x updated, h = next pre-norm of x).
// Decode uses the fused router and route-indexed experts where the sizes
// allow; a prefill always takes router -> permutation -> grouped experts.
// `parts` (decode, fused router only): nparts partial products of the mixer's
// output projection that the router folds into x first (times `gate` if set).
// With the context-aware router the ids and gates come from context_route.
void moe_block(const Model& m, const Layer& L, Buffers& b, int rows, const float* next_norm,
               bool sequence, hipStream_t st, float* ring, const int32_t* pos, int nseq,
               const float* parts = nullptr, int nparts = 0, const float* gate = nullptr,
               const LayerState* ls = nullptr) {
  const Config& c = m.cfg;
  const int D = c.d_model, E = c.experts, k = c.top_k, Hf = c.hidden_p();
  const int kx = c.routes(), EX = c.all_experts();
  const bool fused = !sequence && fused_route(c, rows);
  if (nparts > 0 && !fused) throw std::logic_error("partial products need the fused router");
  // the router's [rows, k] routes, extended by the always-on shared experts
  auto with_shared = [&](const int32_t*& ids, const float*& gts) {
    ids = b.idx;
    gts = b.gates;
    if (c.shared == 0) return;
    check_call(llmy_moe_append_shared(b.idx, b.gates, b.idx_all, b.gates_all, rows, k, E, c.shared,
                                      st),
               "llmy_moe_append_shared");
    ids = b.idx_all;
    gts = b.gates_all;
  };
  const int32_t* ids = nullptr;
  const float* gts = nullptr;
  if (fused) {
    check_call(llmy_moe_route_decode(b.x, parts, nparts, gate, L.ffn_norm, L.router_norm,
                                     L.w_router, b.h, b.idx, b.gates, nullptr, nullptr, nullptr,
                                     nullptr, rows, D, E, k, c.eps, st),
               "llmy_moe_route_decode");
    if (c.ctx) context_route(m, L, b, rows, ring, pos, nseq, ls, st);
    with_shared(ids, gts);
    check_call(llmy_moe_experts_routed_bf16(b.h, ids, gts, L.w_gate_up, L.w_down, b.act, b.y,
                                            rows, D, Hf, EX, kx, kPacked, st),
               "llmy_moe_experts_routed_bf16");
    check_call(llmy_moe_combine_norm(b.y, nullptr, next_norm, b.x, b.h, rows, D, kx, c.eps, st),
               "llmy_moe_combine_norm");
    return;
  }
  if (router_fusable(c)) {  // one launch per token: pre-MoE norm + router + top-k
    check_call(llmy_moe_route_decode(b.x, nullptr, 0, nullptr, L.ffn_norm, L.router_norm,
                                     L.w_router, b.h, b.idx, b.gates, nullptr, nullptr, nullptr,
                                     nullptr, rows, D, E, k, c.eps, st),
               "llmy_moe_route_decode");
  } else {
    check_call(llmy_rmsnorm_f32_bf16(b.x, L.ffn_norm, b.h, rows, D, c.eps, st), "rmsnorm");
    check_call(llmy_router_topk_bf16(b.h, L.router_norm, L.w_router, nullptr, b.idx, b.gates,
                                     rows, D, E, k, c.eps, st),
               "llmy_router_topk_bf16");
  }
  if (c.ctx) context_route(m, L, b, rows, ring, pos, nseq, ls, st);
  with_shared(ids, gts);
  check_call(llmy_moe_permute(ids, rows * kx, EX, b.counts, b.offsets, b.sorted, b.route_pos,
                              st),
             "llmy_moe_permute");
  check_call(llmy_moe_experts_bf16(b.h, b.offsets, b.sorted, gts, L.w_gate_up, L.w_down, b.act,
                                   b.y, rows, D, Hf, EX, kx, kPacked, st),
             "llmy_moe_experts_bf16");
  check_call(llmy_moe_combine_norm(b.y, b.route_pos, next_norm, b.x, b.h, rows, D, kx, c.eps,
                                   st),
             "llmy_moe_combine_norm");
}

// The dense SwiGLU FFN of a stem / tail block (dense_ffn.py:14-15) on b.h: the
// MoE kernels over its one-expert stack with every row routed to it at gate 1
// (decode: route-indexed; prefill: permutation + grouped GEMMs), then added to
// x with h = the next pre-norm (u == nullptr), or stored to u (mHC).
void dense_block(const Model& m, const Layer& L, Buffers& b, int rows, bool sequence,
                 const float* next_norm, float* u, hipStream_t st) {
  const Config& c = m.cfg;
  const int D = c.d_model, Hd = c.dense_p();
  const int32_t* route_pos = nullptr;
  if (!sequence) {
    check_call(llmy_moe_experts_routed_bf16(b.h, b.dids, b.dgates, L.ffn_gate_up, L.ffn_down,
                                            b.dact, b.y, rows, D, Hd, 1, 1, kPacked, st),
               "llmy_moe_experts_routed_bf16 (dense)");
  } else {
    check_call(llmy_moe_permute(b.dids, rows, 1, b.counts, b.offsets, b.sorted, b.route_pos, st),
               "llmy_moe_permute (dense)");
    check_call(llmy_moe_experts_bf16(b.h, b.offsets, b.sorted, b.dgates, L.ffn_gate_up,
                                     L.ffn_down, b.dact, b.y, rows, D, Hd, 1, 1, kPacked, st),
               "llmy_moe_experts_bf16 (dense)");
    route_pos = b.route_pos;
  }
  if (u == nullptr)
    check_call(llmy_moe_combine_norm(b.y, route_pos, next_norm, b.x, b.h, rows, D, 1, c.eps, st),
               "llmy_moe_combine_norm (dense)");
  else
    check_call(llmy_moe_combine(b.y, route_pos ? route_pos : b.mident, u, rows, D, 1, 1, st),
               "llmy_moe_combine (dense)");
}

// The blocks a token passes in order: the stem, the core `loops` times (one
// state per (loop, layer)), the tail (model.py:842-909).
struct App {
  const Layer* L;
  LayerState* st;
};

std::vector<App> apps_of(const Model& m, State& s, int loops) {
  std::vector<App> a;
  const size_t n = m.layers.size();
  for (size_t i = 0; i < m.stem.size(); ++i) a.push_back({&m.stem[i], &s.side[i]});
  for (int loop = 0; loop < loops; ++loop)
    for (size_t l = 0; l < n; ++l) a.push_back({&m.layers[l], &s.layers[loop * n + l]});
  for (size_t i = 0; i < m.tail.size(); ++i)
    a.push_back({&m.tail[i], &s.side[m.stem.size() + i]});
  return a;
}

const float* next_norm_of(const Model& m, const std::vector<App>& a, size_t i) {
  return i + 1 < a.size() ? a[i + 1].L->mix_norm : m.final_norm;
}

// ------------------------------------------------------------------ CSA / HCA
// The compressed-memory mixers (model/layers/csa.py, hca.py).  Kernels and
// their order are the Python engine's (HybridDecoder._cmp / _cmp_seq), so the
// two engines agree bit for bit.  The mixer's output goes to `out` through
// the epilogue `epi` (residual add into x, or a store into mHC's U).

// The router's [k | v] of `n` summary values (rows of kv at kv_ld, value part
// at column Kw) into b.g_kvr: copied dense, LayerNorm(down . value) (hca_latent,
// eps 1e-5), then the latent attention's k | v (model.py:318-334).
void router_summary_kv(const Model& m, const Layer& L, Buffers& b, const uint16_t* vals,
                       int64_t vals_ld, int n, hipStream_t s) {
  const Config& c = m.cfg;
  const int D = c.d_model, Lc = c.latent, Lp = c.latent_p();
  check_call(llmy_cmp_ring_fill_bf16(vals, vals_ld, b.g_val, n, 1, 1, D, s), "summary values");
  linear(b.g_val, L.hca_lat_down, b.g_lat_raw, nullptr, n, Lc, D, kStoreF32, s);
  check_call(llmy_layernorm_f32_bf16(b.g_lat_raw, L.hca_lat_ln_w, L.hca_lat_ln_b, b.g_lat, n, Lc,
                                     1e-5f, s),
             "llmy_layernorm_f32_bf16");
  const uint16_t* lat = b.g_lat;
  if (Lp != Lc) {
    check_call(llmy_pad_cols_bf16(b.g_lat, b.g_lat_p, n, Lc, Lp, s), "llmy_pad_cols_bf16");
    lat = b.g_lat_p;
  }
  linear(lat, L.ctx_kv, b.g_kvr, nullptr, n, 2 * c.hq(), Lp, kStoreBf16, s);
}

// Decode, one token per row at positions pos: q | k | v, the local window over
// the ring (new key / value stored first), the compressor step and the commit
// of completed blocks' summaries, the memory branch, out(local_out + remote_out).
void cmp_decode(const Model& m, const Layer& L, LayerState& st, Buffers& b, int B,
                const int32_t* pos, void* out, int epi, hipStream_t s) {
  const Config& c = m.cfg;
  const CmpShape cs = c.cmp(L.kind);
  const int D = c.d_model, Kw = cs.kw(), N = 2 * Kw + D, C = c.cmp_slots;
  const float scale = 1.0f / std::sqrt(static_cast<float>(cs.Dh));
  linear(b.h, L.cmp_wqkv, b.cqkv, nullptr, B, N, D, kStoreBf16, s);
  check_call(llmy_cmp_local_decode_bf16(b.cqkv, N, b.cqkv + Kw, b.cqkv + 2 * Kw, N, st.lk, st.lv,
                                        pos, b.cloc, 2 * D, B, cs.H, cs.Dh, D, cs.W, scale, b.cws,
                                        b.cws_bytes, s),
             "llmy_cmp_local_decode_bf16");
  check_call(llmy_cmp_pool_step_bf16(b.h, D, st.psum, st.pcnt, b.cmean, b.cemit, B, D, cs.ratio,
                                     s),
             "llmy_cmp_pool_step_bf16");
  linear(b.cmean, L.cmp_wc, b.ckv, nullptr, B, Kw + D, D, kStoreBf16, s);
  check_call(llmy_cmp_commit_bf16(b.ckv, Kw + D, b.cemit, pos, st.mk, st.mv, st.mtag, st.mcount,
                                  B, C, Kw, D, s),
             "llmy_cmp_commit_bf16");
  if (st.rk) {
    router_summary_kv(m, L, b, b.ckv + Kw, Kw + D, B, s);
    check_call(llmy_cmp_commit_bf16(b.g_kvr, 2 * c.hq(), b.cemit, pos, st.rk, st.rv, st.rtag,
                                    st.rcount, B, C, c.hq(), c.hq(), s),
               "llmy_cmp_commit_bf16 (router)");
  }
  check_call(llmy_cmp_memory_decode_bf16(b.cqkv, N, st.mk, st.mv, st.mtag, pos, b.cloc + D, 2 * D,
                                         B, C, cs.H, cs.Dh, D, cs.top_k, scale, b.cws, b.cws_bytes,
                                         s),
             "llmy_cmp_memory_decode_bf16");
  linear(b.cloc, L.cmp_wlr, b.cy, nullptr, B, D, 2 * D, kStoreBf16, s);
  linear(b.cy, L.cmp_wout, out, nullptr, B, D, D, epi, s);
}

// Prefill of B fresh sequences of T tokens: the branches over all rows, the
// block means and their summaries, then the state T decode steps leave.
void cmp_prefill(const Model& m, const Layer& L, LayerState& st, Buffers& b, int B, int T,
                 void* out, int epi, hipStream_t s) {
  const Config& c = m.cfg;
  const CmpShape cs = c.cmp(L.kind);
  const int D = c.d_model, Kw = cs.kw(), N = 2 * Kw + D, C = c.cmp_slots, R = B * T;
  const int n = T / cs.ratio;
  const float scale = 1.0f / std::sqrt(static_cast<float>(cs.Dh));
  linear(b.h, L.cmp_wqkv, b.cqkv, nullptr, R, N, D, kStoreBf16, s);
  check_call(llmy_cmp_local_prefill_bf16(b.cqkv, N, b.cqkv + Kw, N, b.cqkv + 2 * Kw, N, b.cloc,
                                         2 * D, B, T, cs.H, cs.Dh, D, cs.W, scale, b.cws,
                                         b.cws_bytes, s),
             "llmy_cmp_local_prefill_bf16");
  check_call(llmy_cmp_pool_prefill_bf16(b.h, D, b.cmean, st.psum, st.pcnt, B, T, D, cs.ratio, s),
             "llmy_cmp_pool_prefill_bf16");
  if (n > 0) linear(b.cmean, L.cmp_wc, b.ckv, nullptr, B * n, Kw + D, D, kStoreBf16, s);
  check_call(llmy_cmp_memory_prefill_bf16(b.cqkv, N, b.ckv, Kw + D, b.ckv + Kw, Kw + D,
                                          b.cloc + D, 2 * D, B, T, n, cs.ratio, cs.H, cs.Dh, D,
                                          cs.top_k, C, scale, b.cws, b.cws_bytes, s),
             "llmy_cmp_memory_prefill_bf16");
  check_call(llmy_cmp_memory_fill_bf16(b.ckv, Kw + D, st.mk, st.mv, st.mtag, st.mcount, B, n,
                                       cs.ratio, C, Kw, D, s),
             "llmy_cmp_memory_fill_bf16");
  if (st.rk && n > 0) {
    router_summary_kv(m, L, b, b.ckv + Kw, Kw + D, B * n, s);
    check_call(llmy_cmp_memory_fill_bf16(b.g_kvr, 2 * c.hq(), st.rk, st.rv, st.rtag, st.rcount, B,
                                         n, cs.ratio, C, c.hq(), c.hq(), s),
               "llmy_cmp_memory_fill_bf16 (router)");
  }
  check_call(llmy_cmp_ring_fill_bf16(b.cqkv + Kw, N, st.lk, B, T, cs.W, Kw, s), "ring fill k");
  check_call(llmy_cmp_ring_fill_bf16(b.cqkv + 2 * Kw, N, st.lv, B, T, cs.W, D, s), "ring fill v");
  linear(b.cloc, L.cmp_wlr, b.cy, nullptr, R, D, 2 * D, kStoreBf16, s);
  linear(b.cy, L.cmp_wout, out, nullptr, R, D, D, epi, s);
}

// ------------------------------------------------------------------ mHC
// Multi-stream hyper-connections around each sublayer (model/model.py:119-126,
// 177-264; model/layers/mhc.py:156-231).  The kernels and their order are the
// Python engine's (HybridDecoder._step_body_mhc / _prefill_mhc), so the two
// engines agree bit for bit.
constexpr float kMhcMapEps = 1.1920928955078125e-07f;  // nn.RMSNorm(eps=None), fp32

// The sublayer input of layer L from the streams: maps into b.mmaps, h into b.h.
void mhc_read(const Model& m, const Layer& L, Buffers& b, int rows, const float* norm,
              hipStream_t st) {
  const Config& c = m.cfg;
  const int S = c.mhc, D = c.d_model;
  check_call(llmy_rmsnorm_f32_bf16(b.mX, L.mhc_map_norm, b.mxb, rows, S * D, kMhcMapEps, st),
             "llmy_rmsnorm_f32_bf16 (mHC)");
  linear(b.mxb, L.mhc_theta, b.mraw, nullptr, rows, c.mhc_n16(), S * D, kStoreF32, st);
  check_call(llmy_mhc_read(b.mX, b.mraw, c.mhc_n16(), L.mhc_pre_bias, L.mhc_post_bias,
                           L.mhc_res_bias, L.mhc_alpha, c.mhc_iters, L.mhc_ln_w, L.mhc_ln_b, 1e-5f,
                           norm, c.eps, b.mmaps, b.h, rows, S, D, st),
             "llmy_mhc_read");
}

void mhc_write(const Model& m, const Layer& L, Buffers& b, int rows, hipStream_t st) {
  check_call(llmy_mhc_write(b.mX, b.mU, m.cfg.d_model, b.mmaps, L.mhc_scale, L.mhc_gating, rows,
                            m.cfg.mhc, m.cfg.d_model, st),
             "llmy_mhc_write");
}

void mhc_clear_u(const Model& m, Buffers& b, int rows, hipStream_t st) {
  check_call(llmy_zero_rows(b.mU, static_cast<int64_t>(m.cfg.d_model) * 4, rows, b.mones, st),
             "llmy_zero_rows");
}

// The MoE of layer L on b.h into U: router + top-k, then route-indexed experts
// (decode, where the sizes allow) or permutation + grouped experts.
void mhc_moe(const Model& m, const Layer& L, Buffers& b, int rows, bool sequence, hipStream_t st,
             float* ring, const int32_t* pos, int nseq, const LayerState* ls) {
  const Config& c = m.cfg;
  const int D = c.d_model, E = c.experts, k = c.top_k, Hf = c.hidden_p();
  const int kx = c.routes(), EX = c.all_experts();
  if (c.ctx)
    context_route(m, L, b, rows, ring, pos, nseq, ls, st);
  else
    check_call(llmy_router_topk_bf16(b.h, L.router_norm, L.w_router, nullptr, b.idx, b.gates,
                                     rows, D, E, k, c.eps, st),
               "llmy_router_topk_bf16");
  const int32_t* ids = b.idx;
  const float* gts = b.gates;
  if (c.shared > 0) {
    check_call(llmy_moe_append_shared(b.idx, b.gates, b.idx_all, b.gates_all, rows, k, E,
                                      c.shared, st),
               "llmy_moe_append_shared");
    ids = b.idx_all;
    gts = b.gates_all;
  }
  const int32_t* route_pos = b.mident;
  if (!sequence && fused_route(c, rows)) {
    check_call(llmy_moe_experts_routed_bf16(b.h, ids, gts, L.w_gate_up, L.w_down, b.act, b.y,
                                            rows, D, Hf, EX, kx, kPacked, st),
               "llmy_moe_experts_routed_bf16");
  } else {
    check_call(llmy_moe_permute(ids, rows * kx, EX, b.counts, b.offsets, b.sorted, b.route_pos,
                                st),
               "llmy_moe_permute");
    check_call(llmy_moe_experts_bf16(b.h, b.offsets, b.sorted, gts, L.w_gate_up, L.w_down, b.act,
                                     b.y, rows, D, Hf, EX, kx, kPacked, st),
               "llmy_moe_experts_bf16");
    route_pos = b.route_pos;
  }
  check_call(llmy_moe_combine(b.y, route_pos, b.mU, rows, D, kx, 1, st), "llmy_moe_combine");
}

// Collapse the streams, final RMSNorm, LM head, argmax (model.py:699-705).
void mhc_head(const Model& m, State& s, Buffers& b, int rows, hipStream_t st) {
  const Config& c = m.cfg;
  const int S = c.mhc, D = c.d_model;
  check_call(llmy_f32_to_bf16(b.mX, b.mxb, static_cast<int64_t>(rows) * S * D, st),
             "llmy_f32_to_bf16");
  linear(b.mxb, m.mhc_collapse, b.mU, nullptr, rows, D, S * D, kStoreF32, st);
  check_call(llmy_rmsnorm_f32_bf16(b.mU, m.final_norm, b.h, rows, D, c.eps, st), "rmsnorm");
  linear(b.h, m.lm_head, s.logits, nullptr, rows, c.vocab, D, kStoreF32, st);
  check_call(llmy_sample_argmax_f32(s.logits, rows, c.vocab, s.next, st), "argmax");
}

// The attention mixer of one decode token per row into `out` (epilogue epi),
// or, with `parts`, its output projection as per-K-block partial products.
void attn_decode(const Model& m, const Layer& L, LayerState& st, Buffers& b, int B,
                 const int32_t* pos, void* out, int epi, hipStream_t s) {
  const Config& c = m.cfg;
  const int D = c.d_model, Hhd = c.attn_heads * c.attn_head_dim;
  const float scale = 1.0f / std::sqrt(static_cast<float>(c.attn_head_dim));
  if (b.qkv_parts != nullptr) {
    // q/k/v as partial products, summed and rounded by the attention kernel
    linear(b.h, L.wqkv, b.qkv_parts, nullptr, B, 3 * Hhd, D, kPartialF32, s);
    check_call(llmy_banded_attn_decode_parts_bf16(b.qkv_parts, D / 256,
                                                  static_cast<int64_t>(B) * 3 * Hhd, 3 * Hhd, Hhd,
                                                  2 * Hhd, st.k, st.v, pos, b.ao, B,
                                                  c.attn_heads, c.attn_head_dim, c.window, scale,
                                                  s),
               "llmy_banded_attn_decode_parts_bf16");
  } else {
    linear(b.h, L.wqkv, b.qkv, nullptr, B, 3 * Hhd, D, kStoreBf16, s);
    check_call(llmy_banded_attn_decode_bf16(b.qkv, b.qkv + Hhd, b.qkv + 2 * Hhd, 3 * Hhd,
                                            3 * Hhd, st.k, st.v, pos, b.ao, B, c.attn_heads,
                                            c.attn_head_dim, c.window, scale, s),
               "llmy_banded_attn_decode_bf16");
  }
  linear(b.ao, L.wo, out, nullptr, B, D, Hhd, epi, s);
}

// The GDN mixer of one decode token per row: the input projection (as partial
// products summed by the step kernel at small batches), the fused step, then
// the output projection gated by the conv into `out` (epilogue epi: residual
// add into x or U, or kPartialF32 into b.parts).
void gdn_decode(const Model& m, const Layer& L, LayerState& st, Buffers& b, int B, void* out,
                int epi, hipStream_t s) {
  const Config& c = m.cfg;
  const int D = c.d_model, HV = c.gdn_heads * c.dv;
  const bool pp = b.proj_parts != nullptr;
  float* proj = pp ? b.proj_parts : b.proj;
  linear(b.h, L.wproj, proj, nullptr, B, c.nproj16(), D, pp ? kPartialF32 : kStoreF32, s);
  check_call(llmy_gdn_step_fused_f32(proj, c.nproj16(), pp ? D / 256 : 1, L.bb, L.decay, st.S,
                                     b.go, b.h, st.hist, L.conv, b.cg, D, 4, B, c.gdn_heads, c.dk,
                                     c.dv, s),
             "llmy_gdn_step_fused_f32");
  linear(b.go, L.wout, out, epi == kPartialF32 ? nullptr : b.cg, B, D, HV, epi, s);
}

// The attention mixer over B fresh sequences of T tokens, into `out` (epi),
// then the last min(T, W) keys / values into the ring caches.
void attn_prefill(const Model& m, const Layer& L, LayerState& st, Buffers& b, int B, int T,
                  void* out, int epi, hipStream_t s) {
  const Config& c = m.cfg;
  const int D = c.d_model, R = B * T, Hhd = c.attn_heads * c.attn_head_dim;
  // q, k, v from row slices of the packed wqkv (each a packed [Hhd, D] matrix)
  const size_t slice = static_cast<size_t>(Hhd) * D;
  linear(b.h, L.wqkv, b.q, nullptr, R, Hhd, D, kStoreBf16, s);
  linear(b.h, L.wqkv + slice, b.k, nullptr, R, Hhd, D, kStoreBf16, s);
  linear(b.h, L.wqkv + 2 * slice, b.v, nullptr, R, Hhd, D, kStoreBf16, s);
  check_call(llmy_banded_attn_prefill_bf16(b.q, b.k, b.v, b.ao, B, T, c.attn_heads,
                                           c.attn_head_dim, c.window,
                                           1.0f / std::sqrt(static_cast<float>(c.attn_head_dim)),
                                           s),
             "llmy_banded_attn_prefill_bf16");
  check_call(llmy_kv_cache_fill_bf16(b.k, b.v, Hhd, st.k, st.v, B, T, c.attn_heads,
                                     c.attn_head_dim, c.window, s),
             "llmy_kv_cache_fill_bf16");
  linear(b.ao, L.wo, out, nullptr, R, D, Hhd, epi, s);
}

// The GDN mixer over B fresh sequences of T tokens, gated by the conv and
// added to `out` (x, or the cleared U).
void gdn_prefill(const Model& m, const Layer& L, LayerState& st, Buffers& b, int B, int T,
                 float* out, hipStream_t s) {
  const Config& c = m.cfg;
  const int D = c.d_model, R = B * T, H = c.gdn_heads, HV = H * c.dv;
  linear(b.h, L.wproj, b.proj, nullptr, R, c.nproj16(), D, kStoreF32, s);
  check_call(llmy_gdn_prefill_prep_f32(b.proj, c.nproj16(), L.bb, L.decay, b.gq, b.gk, b.gv,
                                       b.beta, b.g, R, H, c.dk, c.dv, s),
             "llmy_gdn_prefill_prep_f32");
  check_call(llmy_gdn_prefill_bf16(b.gq, b.gk, b.gv, b.beta, b.g, st.S, b.go, b.ws, b.ws_bytes, B,
                                   T, H, c.dk, c.dv, s),
             "llmy_gdn_prefill_bf16");
  check_call(llmy_gdn_gate_bf16(b.go, b.proj, c.nproj16(), 2 * H * c.dk + HV, b.go, R, HV, s),
             "llmy_gdn_gate_bf16");
  check_call(llmy_gdn_conv_gate_prefill(b.h, st.hist, L.conv, b.cg, B, T, D, 4, s),
             "llmy_gdn_conv_gate_prefill");
  linear(b.go, L.wout, out, b.cg, R, D, HV, kResidGated, s);
}

void decode_step_mhc(Model& m, State& s, int loops) {
  hipStream_t st_ = s.stream;
  const Config& c = m.cfg;
  Buffers& b = s.step;
  const int B = s.B, D = c.d_model;
  check_call(llmy_mhc_embed(b.tokens, m.embed, m.stream_seed, b.mX, B, c.mhc, D, c.vocab, st_),
             "llmy_mhc_embed");
  for (const App& a : apps_of(m, s, loops)) {
    const Layer& L = *a.L;
    LayerState& st = *a.st;
    mhc_read(m, L, b, B, L.mix_norm, st_);
    if (L.kind == kAttn) {
      attn_decode(m, L, st, b, B, s.pos, b.mU, kStoreF32, st_);
    } else if (L.kind == kCsa || L.kind == kHca) {
      cmp_decode(m, L, st, b, B, s.pos, b.mU, kStoreF32, st_);
    } else {
      mhc_clear_u(m, b, B, st_);
      gdn_decode(m, L, st, b, B, b.mU, kResidGated, st_);
    }
    mhc_write(m, L, b, B, st_);
    mhc_read(m, L, b, B, L.ffn_norm, st_);
    if (L.side)
      dense_block(m, L, b, B, false, nullptr, b.mU, st_);
    else
      mhc_moe(m, L, b, B, false, st_, st.ring, s.pos, B, &st);
    mhc_write(m, L, b, B, st_);
  }
  mhc_head(m, s, b, B, st_);
  s.last_loops = loops;
}

// One decode step for all B rows; tokens already in s.step.tokens, s.pos set.
void decode_step(Model& m, State& s, int loops) {
  if (m.cfg.mhc > 1) {
    decode_step_mhc(m, s, loops);
    return;
  }
  hipStream_t st_ = s.stream;
  const Config& c = m.cfg;
  Buffers& b = s.step;
  const int B = s.B, D = c.d_model;
  const std::vector<App> apps = apps_of(m, s, loops);
  check_call(llmy_embed_norm_bf16(b.tokens, m.embed, apps[0].L->mix_norm, b.x, b.h, B, D, c.vocab,
                                  c.eps, st_),
             "llmy_embed_norm_bf16");
  const int Hhd = c.attn_heads * c.attn_head_dim, HV = c.gdn_heads * c.dv;
  // core mixers' output projections as partial products folded by the router
  const bool defer = b.parts != nullptr && fused_route(c, B);
  for (size_t i = 0; i < apps.size(); ++i) {
    const Layer& L = *apps[i].L;
    LayerState& st = *apps[i].st;
    const float* next = next_norm_of(m, apps, i);
    if (L.side) {  // GDN into x, the dense FFN's pre-norm, the FFN
      gdn_decode(m, L, st, b, B, b.x, kResidGated, st_);
      check_call(llmy_rmsnorm_f32_bf16(b.x, L.ffn_norm, b.h, B, D, c.eps, st_), "rmsnorm");
      dense_block(m, L, b, B, false, next, nullptr, st_);
      continue;
    }
    int nparts = 0;
    const float* gate = nullptr;
    if (L.kind == kAttn) {
      attn_decode(m, L, st, b, B, s.pos, defer ? static_cast<void*>(b.parts) : b.x,
                  defer ? kPartialF32 : kResidAdd, st_);
      nparts = defer ? Hhd / 256 : 0;
    } else if (L.kind == kCsa || L.kind == kHca) {
      cmp_decode(m, L, st, b, B, s.pos, b.x, kResidAdd, st_);
    } else {
      gdn_decode(m, L, st, b, B, defer ? static_cast<void*>(b.parts) : b.x,
                 defer ? kPartialF32 : kResidGated, st_);
      nparts = defer ? HV / 256 : 0;
      gate = defer ? b.cg : nullptr;
    }
    moe_block(m, L, b, B, next, false, st_, st.ring, s.pos, B, b.parts, nparts, gate, &st);
  }
  linear(b.h, m.lm_head, s.logits, nullptr, B, c.vocab, D, kStoreF32, st_);
  check_call(llmy_sample_argmax_f32(s.logits, B, c.vocab, s.next, st_), "argmax");
  s.last_loops = loops;
}

// Prefill with mHC: the sequence kernels of prefill() with each sublayer's
// output in U, written into the [B T, S, D] streams (tokens already in b).
void prefill_mhc(Model& m, State& s, Buffers& b, int T) {
  hipStream_t st_ = s.stream;
  const Config& c = m.cfg;
  const int B = s.B, R = B * T, D = c.d_model, S = c.mhc;
  check_call(llmy_mhc_embed(b.tokens, m.embed, m.stream_seed, b.mX, R, S, D, c.vocab, st_),
             "llmy_mhc_embed");
  const int loops = m.loops;
  for (const App& a : apps_of(m, s, loops)) {
    const Layer& L = *a.L;
    LayerState& st = *a.st;
    mhc_read(m, L, b, R, L.mix_norm, st_);
    if (L.kind == kAttn) {
      attn_prefill(m, L, st, b, B, T, b.mU, kStoreF32, st_);
    } else if (L.kind == kCsa || L.kind == kHca) {
      cmp_prefill(m, L, st, b, B, T, b.mU, kStoreF32, st_);
    } else {
      mhc_clear_u(m, b, R, st_);
      gdn_prefill(m, L, st, b, B, T, b.mU, st_);
    }
    mhc_write(m, L, b, R, st_);
    mhc_read(m, L, b, R, L.ffn_norm, st_);
    if (L.side)
      dense_block(m, L, b, R, true, nullptr, b.mU, st_);
    else
      mhc_moe(m, L, b, R, true, st_, st.ring, nullptr, B, &st);
    mhc_write(m, L, b, R, st_);
  }
  // each sequence's last streams -> the decode buffers, then the head
  const size_t row = static_cast<size_t>(S) * D * 4;
  check_hip(hipMemcpy2DAsync(s.step.mX, row, b.mX + static_cast<size_t>(T - 1) * S * D, T * row,
                             row, B, hipMemcpyDeviceToDevice, st_),
            "last streams");
  mhc_head(m, s, s.step, B, st_);
  s.hpos.assign(B, T);
  check_hip(hipMemcpyAsync(s.pos, s.hpos.data(), sizeof(int32_t) * B, hipMemcpyHostToDevice, st_),
            "pos");
  check_hip(hipStreamSynchronize(st_), "prefill");
  s.last_loops = loops;
}

// Prefill of B fresh sequences of T tokens each (tokens on the host, [B, T]).
void prefill(Model& m, State& s, const int32_t* tokens, int T, bool tokens_on_device) {
  hipStream_t st_ = s.stream;
  const Config& c = m.cfg;
  const int B = s.B, R = B * T, D = c.d_model;
  // prompts the compressed-memory prefill cannot take are refused before any
  // kernel runs (the Python engine's check_prompt_length)
  for (int kind : {kCsa, kHca}) {
    if (!c.has(kind)) continue;
    const int ratio = c.cmp(kind).ratio, n = T / ratio;
    if (n > 4000)
      throw std::runtime_error("prompt too long: a CSA / HCA block's prefill takes at most 4000 "
                               "summaries per row");
    if (kind == kHca && c.ctx && n > c.cmp_slots)
      throw std::runtime_error("prompt emits more HCA summaries per row than the router's summary "
                               "memory keeps (memory.decode_slots)");
  }
  reset_state(s);
  if (!s.seq || s.seq->rows < R || (c.has_gdn() && s.seq->ws_bytes <
                                    llmy_gdn_prefill_workspace_bytes(B, T, c.gdn_heads, c.dk, c.dv))) {
    s.seq.reset();
    auto nb = std::make_unique<Buffers>();
    alloc_buffers(c, R, B, std::max(T, 2), *nb);
    s.seq = std::move(nb);
  }
  Buffers& b = *s.seq;
  check_hip(hipMemcpyAsync(b.tokens, tokens, sizeof(int32_t) * R,
                           tokens_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, st_),
            "tokens");
  if (c.mhc > 1) {
    prefill_mhc(m, s, b, T);
    return;
  }
  // the loop count set by llmy_set_num_loops (model_prefill runs cfg.num_loops,
  // which llmy_set_num_loops overwrites: llmy_cuda/src/model.cpp:1964, llmy.cpp:66-69)
  const int loops = m.loops;
  const std::vector<App> apps = apps_of(m, s, loops);
  check_call(llmy_embed_norm_bf16(b.tokens, m.embed, apps[0].L->mix_norm, b.x, b.h, R, D, c.vocab,
                                  c.eps, st_),
             "llmy_embed_norm_bf16");
  for (size_t i = 0; i < apps.size(); ++i) {
    const Layer& L = *apps[i].L;
    LayerState& st = *apps[i].st;
    const float* next = next_norm_of(m, apps, i);
    if (L.side) {
      gdn_prefill(m, L, st, b, B, T, b.x, st_);
      check_call(llmy_rmsnorm_f32_bf16(b.x, L.ffn_norm, b.h, R, D, c.eps, st_), "rmsnorm");
      dense_block(m, L, b, R, true, next, nullptr, st_);
      continue;
    }
    if (L.kind == kAttn)
      attn_prefill(m, L, st, b, B, T, b.x, kResidAdd, st_);
    else if (L.kind == kCsa || L.kind == kHca)
      cmp_prefill(m, L, st, b, B, T, b.x, kResidAdd, st_);
    else
      gdn_prefill(m, L, st, b, B, T, b.x, st_);
    moe_block(m, L, b, R, next, true, st_, st.ring, nullptr, B, nullptr, 0, nullptr, &st);
  }
  // last position of each sequence -> the decode buffer, then the LM head
  check_hip(hipMemcpy2DAsync(s.step.h, static_cast<size_t>(D) * 2,
                             b.h + static_cast<size_t>(T - 1) * D, static_cast<size_t>(T) * D * 2,
                             static_cast<size_t>(D) * 2, B, hipMemcpyDeviceToDevice, st_),
            "last rows");
  linear(s.step.h, m.lm_head, s.logits, nullptr, B, c.vocab, D, kStoreF32, st_);
  check_call(llmy_sample_argmax_f32(s.logits, B, c.vocab, s.next, st_), "argmax");
  s.hpos.assign(B, T);
  check_hip(hipMemcpyAsync(s.pos, s.hpos.data(), sizeof(int32_t) * B, hipMemcpyHostToDevice, st_),
            "pos");
  check_hip(hipStreamSynchronize(st_), "prefill");
  s.last_loops = loops;
}

void copy_logits_out(const State& s, float* out) {
  const size_t bytes = sizeof(float) * s.B * s.model->cfg.vocab;
  check_hip(hipMemcpyAsync(out, s.logits, bytes, hipMemcpyDefault, s.stream), "logits");
  check_hip(hipStreamSynchronize(s.stream), "logits");
}

// The decode step for `loops` loops as one graph launch: captured on the
// state's stream the first time (kernels only, no memory set or copy), then
// replayed.  Token ids and positions live in device buffers the graph reads.
void run_decode(Model& m, State& s, int loops) {
  auto it = s.graphs.find(loops);
  if (it == s.graphs.end()) {
    hipGraph_t g = nullptr;
    check_hip(hipStreamBeginCapture(s.stream, hipStreamCaptureModeRelaxed), "begin capture");
    try {
      decode_step(m, s, loops);
    } catch (...) {
      (void)hipStreamEndCapture(s.stream, &g);
      if (g) (void)hipGraphDestroy(g);
      throw;
    }
    check_hip(hipStreamEndCapture(s.stream, &g), "end capture");
    hipGraphExec_t exec = nullptr;
    const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    check_hip(e, "graph instantiate");
    it = s.graphs.emplace(loops, exec).first;
  }
  check_hip(hipGraphLaunch(it->second, s.stream), "graph launch");
  s.last_loops = loops;
}

Model* as_model(llmy_model* p) { return reinterpret_cast<Model*>(p); }
State* as_state(llmy_state* p) { return reinterpret_cast<State*>(p); }

template <typename F>
int32_t guarded(F&& f) {
  try {
    f();
    g_status = 0;
    g_error[0] = '\0';
    return 0;
  } catch (const std::exception& e) {
    set_error(1, e.what());
    std::fprintf(stderr, "[llmy] %s\n", e.what());
    return 1;
  }
}

}  // namespace

// ================================================================== C ABI
extern "C" {

llmy_model* llmy_load(const char* path) {
  if (!path) {
    set_error(1, "null path");
    return nullptr;
  }
  Model* out = nullptr;
  guarded([&] { out = load_model(path).release(); });
  return reinterpret_cast<llmy_model*>(out);
}

void llmy_free(llmy_model* m) { delete as_model(m); }

int32_t llmy_vocab_size(const llmy_model* m) {
  return m ? reinterpret_cast<const Model*>(m)->cfg.vocab : 0;
}
int32_t llmy_d_model(const llmy_model* m) {
  return m ? reinterpret_cast<const Model*>(m)->cfg.d_model : 0;
}
int32_t llmy_num_loops(const llmy_model* m) {
  return m ? reinterpret_cast<const Model*>(m)->loops : 0;
}
int32_t llmy_max_loops(const llmy_model* m) {
  return m ? reinterpret_cast<const Model*>(m)->cfg.num_loops : 0;
}
int32_t llmy_mhc_streams(const llmy_model* m) {
  return m ? reinterpret_cast<const Model*>(m)->cfg.mhc : 0;
}

void llmy_set_num_loops(llmy_model* m, int32_t n) {
  if (!m) return;
  Model* mm = as_model(m);
  mm->loops = std::max(1, std::min<int32_t>(n, mm->cfg.num_loops));
}
void llmy_set_fixed_loops(llmy_model* m, int32_t n) {
  if (n >= 1) llmy_set_num_loops(m, n);
}

llmy_state* llmy_state_new(llmy_model* m) { return llmy_state_new_batch(m, 1); }

llmy_state* llmy_state_new_batch(llmy_model* m, int32_t batch) {
  if (!m || batch < 1) {
    set_error(1, "null model or batch < 1");
    return nullptr;
  }
  State* out = nullptr;
  guarded([&] { out = new_state(as_model(m), batch).release(); });
  return reinterpret_cast<llmy_state*>(out);
}

void llmy_state_free(llmy_state* s) { delete as_state(s); }

void llmy_state_reset(llmy_state* s) {
  if (s) guarded([&] { reset_state(*as_state(s)); });
}

void llmy_prefill(llmy_model* m, llmy_state* s, const int32_t* tokens, int32_t n_tokens,
                  float* logits_out) {
  (void)llmy_prefill_batch(m, s, tokens, n_tokens, logits_out);
}

int32_t llmy_prefill_batch(llmy_model* m, llmy_state* s, const int32_t* tokens, int32_t n_tokens,
                           float* logits_out) {
  if (!m || !s || !tokens || n_tokens < 1 || as_state(s)->model != as_model(m)) {
    set_error(1, "invalid prefill arguments");
    return 1;
  }
  return guarded([&] {
    hipPointerAttribute_t attr{};
    const bool on_device = hipPointerGetAttributes(&attr, tokens) == hipSuccess &&
                           attr.type == hipMemoryTypeDevice;
    (void)hipGetLastError();
    prefill(*as_model(m), *as_state(s), tokens, n_tokens, on_device);
    if (logits_out) copy_logits_out(*as_state(s), logits_out);
  });
}

void llmy_decode(llmy_model* m, llmy_state* s, int32_t token, int32_t position, int32_t num_loops,
                 float* logits_out) {
  if (!s || as_state(s)->B != 1) {
    set_error(1, "llmy_decode needs a batch-1 state");
    return;
  }
  (void)llmy_decode_batch(m, s, &token, &position, num_loops, logits_out);
}

int32_t llmy_decode_batch(llmy_model* m, llmy_state* s, const int32_t* tokens,
                          const int32_t* positions, int32_t num_loops, float* logits_out) {
  if (!m || !s || !tokens || as_state(s)->model != as_model(m)) {
    set_error(1, "invalid decode arguments");
    return 1;
  }
  return guarded([&] {
    Model& mm = *as_model(m);
    State& st = *as_state(s);
    // an explicit count is capped at the set one (model.cpp:1824-1825 caps at
    // cfg.num_loops, which llmy_set_num_loops overwrites)
    const int loops = num_loops <= 0 ? mm.loops : std::min<int32_t>(num_loops, mm.loops);
    if (positions)
      check_hip(hipMemcpy(st.hpos.data(), positions, sizeof(int32_t) * st.B, hipMemcpyDefault),
                "positions");
    check_hip(hipMemcpyAsync(st.step.tokens, tokens, sizeof(int32_t) * st.B, hipMemcpyDefault,
                             st.stream),
              "tokens");
    check_hip(hipMemcpyAsync(st.pos, st.hpos.data(), sizeof(int32_t) * st.B,
                             hipMemcpyHostToDevice, st.stream),
              "positions");
    run_decode(mm, st, loops);
    if (logits_out) copy_logits_out(st, logits_out);
    check_hip(hipStreamSynchronize(st.stream), "decode");
    // the next token's position: one past this one (changed only after the
    // stream has drained, so the pageable source of the copy above is stable)
    for (int32_t& p : st.hpos) ++p;
  });
}

int32_t llmy_state_reset_rows(llmy_state* s, const int32_t* mask) {
  if (!s || !mask) {
    set_error(1, "null state or mask");
    return 1;
  }
  return guarded([&] { reset_rows(*as_state(s), mask); });
}

int32_t llmy_greedy_tokens(const llmy_state* s, int32_t* out) {
  if (!s || !out) return 1;
  const State* st = reinterpret_cast<const State*>(s);
  hipError_t e = hipMemcpyAsync(out, st->next, sizeof(int32_t) * st->B, hipMemcpyDefault,
                                st->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(st->stream);
  return static_cast<int32_t>(e);
}

int32_t llmy_sample(const float* logits, int32_t vocab_size, float temperature, int32_t top_k,
                    float top_p, float repetition_penalty, const int32_t* recent_tokens,
                    int32_t n_recent, uint64_t* rng_state) {
  // The CPU sampler of the reference ABI (llmy_cuda/src/llmy.cpp:132-202):
  // penalty per listed id, top-k (capped at 256) by descending logit, greedy
  // for temperature <= 0, softmax / temperature in fp32, the first prefix
  // whose cumulative probability reaches top_p, renormalise, one xorshift64
  // draw u = (r >> 11) / 2^53, the first id whose running sum exceeds u.
  // Equal logits are ordered by ascending id (the twin's partial_sort leaves
  // them unordered).
  if (vocab_size <= 0 || !logits) return 0;
  if (top_k <= 0 || top_k > vocab_size) top_k = vocab_size;
  top_k = std::min(top_k, 256);
  std::vector<float> work(logits, logits + vocab_size);
  if (repetition_penalty != 1.0f && n_recent > 0 && recent_tokens) {
    for (int r = 0; r < n_recent; ++r) {
      const int id = recent_tokens[r];
      if (id < 0 || id >= vocab_size) continue;
      work[id] = work[id] > 0.0f ? work[id] / repetition_penalty : work[id] * repetition_penalty;
    }
  }
  std::vector<int> order(vocab_size);
  for (int i = 0; i < vocab_size; ++i) order[i] = i;
  std::partial_sort(order.begin(), order.begin() + top_k, order.end(), [&](int a, int b) {
    return work[a] > work[b] || (work[a] == work[b] && a < b);
  });
  if (!(temperature > 0.0f)) return order[0];
  const float maxv = work[order[0]];
  std::vector<float> probs(top_k);
  float sum = 0.0f;
  for (int i = 0; i < top_k; ++i) {
    probs[i] = std::exp((work[order[i]] - maxv) / temperature);
    sum += probs[i];
  }
  for (float& p : probs) p /= sum;
  int cutoff = top_k;
  if (top_p > 0.0f && top_p < 1.0f) {
    float cdf = 0.0f;
    for (int i = 0; i < top_k; ++i) {
      cdf += probs[i];
      if (cdf >= top_p) {
        cutoff = i + 1;
        break;
      }
    }
  }
  float renorm = 0.0f;
  for (int i = 0; i < cutoff; ++i) renorm += probs[i];
  for (int i = 0; i < cutoff; ++i) probs[i] /= renorm;
  uint64_t r = rng_state ? *rng_state : 0x9E3779B97F4A7C15ull;
  r ^= r << 13;
  r ^= r >> 7;
  r ^= r << 17;
  if (rng_state) *rng_state = r;
  const double u = static_cast<double>(r >> 11) / static_cast<double>(1ull << 53);
  float acc = 0.0f;
  for (int i = 0; i < cutoff; ++i) {
    acc += probs[i];
    if (u < acc) return order[i];
  }
  return order[cutoff - 1];
}

int32_t llmy_last_executed_loops(const llmy_state* s) {
  return s ? reinterpret_cast<const State*>(s)->last_loops : 0;
}

void llmy_sync(void) { (void)hipDeviceSynchronize(); }

int32_t llmy_last_status(void) { return g_status; }

const char* llmy_last_error(void) { return g_error; }

int32_t llmy_checkpoint_describe(const char* path, char* buf, int64_t buf_len) {
  // Parse only (no device work): config text, then one line per tensor
  // "name dtype ndim d0 d1 d2 d3 nbytes", for hosts without a GPU.
  if (!path || !buf || buf_len < 1) return 1;
  return guarded([&] {
    Checkpoint ck;
    parse_checkpoint(path, ck);
    (void)config_from(ck.config);
    std::string out = ck.config;
    if (!out.empty() && out.back() != '\n') out += '\n';
    out += "--\n";
    for (const auto& kv : ck.tensors) {
      const TensorRef& t = kv.second;
      int64_t d[4] = {0, 0, 0, 0};
      for (size_t i = 0; i < t.shape.size(); ++i) d[i] = t.shape[i];
      char line[160];
      std::snprintf(line, sizeof(line), "%s %u %zu %lld %lld %lld %lld %llu\n", kv.first.c_str(),
                    t.dtype, t.shape.size(), static_cast<long long>(d[0]),
                    static_cast<long long>(d[1]), static_cast<long long>(d[2]),
                    static_cast<long long>(d[3]), static_cast<unsigned long long>(t.nbytes));
      out += line;
    }
    if (static_cast<int64_t>(out.size()) + 1 > buf_len)
      throw std::runtime_error("description buffer too small");
    std::memcpy(buf, out.c_str(), out.size() + 1);
  });
}

}  // extern "C"
