// Host runtime of the t0hip engine: device context, resident GGUF weights,
// per-model workspace and stream, the forward pass as a kernel sequence on
// that stream, the forecast drivers, and every extern "C" entry point of
// include/t0hip.h.
//
// Reference structure this replaces: crates/t0-fast/src/{engine.rs, pool.rs,
// model.rs (GpuModel, forward_async), lib.rs (forecast entry points)}.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <numeric>
#include <string>
#include <unordered_map>
#include <vector>

#include "kernels.h"
#include "t0hip_internal.h"

namespace t0h {

std::vector<uint8_t> synth_model_gguf(const t0h_synth_spec& s, int quant);
std::vector<uint8_t> export_gguf(const uint8_t* bytes, size_t len, int quant);

namespace {
thread_local std::string g_last_error;

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw Error(T0H_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}
}  // namespace

void set_error(const std::string& msg) { g_last_error = msg; }

// ---------------------------------------------------------------------------
// Resident model
// ---------------------------------------------------------------------------
struct Mat {
  const void* w = nullptr;
  int type = T0H_F16;
  int n = 0, k = 0;
  size_t bytes = 0;
};
struct RBlock {  // ops.rs:24-37 residual block
  Mat hid, out, res;
  const float *hb = nullptr, *ob = nullptr, *rb = nullptr;
};
struct Layer {
  bool group = false;
  Mat qkv, o, w0, w2;
  const float *b_qkv, *b_o, *b0, *b2, *norm, *mlp_norm, *q_norm, *k_norm;
  std::vector<float> q_norm_h, k_norm_h;  // host copies, folded into the time-attention tables
};

struct Buf {
  void* p = nullptr;
  size_t cap = 0;
};

// Pinned host staging for one upload stream-ordered on the model's stream; the
// event marks when the last copy out of it has executed.
struct Stage {
  void* p = nullptr;
  size_t cap = 0;
  hipEvent_t ev = nullptr;
  bool pending = false;
};

// A window forward captured as a HIP graph.  It is replayed only while every
// value the captured launches bake in is unchanged: the window shape, the
// longest group segment (which picks the group-attention kernel) and the
// segment count (its grid), the input
// and output pointers and the workspace generation (the allocation count, so
// that a buffer reallocated since the capture is never replayed).
struct GraphKey {
  int v = 0, t_ctx = 0, horizon = 0, seg_max = 0, n_seg = 0;
  const void* ctx = nullptr;
  const void* out = nullptr;
  uint64_t ws_gen = 0;
  bool operator==(const GraphKey& o) const {
    return v == o.v && t_ctx == o.t_ctx && horizon == o.horizon && seg_max == o.seg_max && n_seg == o.n_seg &&
           ctx == o.ctx && out == o.out && ws_gen == o.ws_gen;
  }
};
struct GraphEntry {
  GraphKey key;
  hipGraphExec_t exec = nullptr;  // null: seen once, run eagerly
  uint64_t last_use = 0;
};

struct Workspace {
  std::unordered_map<std::string, Buf> bufs;
  std::unordered_map<std::string, Stage> stages;
  // last bytes uploaded by put_cached per buffer (skipped when unchanged)
  std::unordered_map<std::string, std::vector<uint8_t>> shadow;
  uint64_t allocs = 0;
  int rope_p = -1;
  int seg_max = 0;  // longest group segment of the last upload_segments
  int n_seg = 0;    // and its number of segments
  bool capturing = false;  // a graph capture is recording this model's launches
  bool graphs = true;      // window forwards are captured and replayed
  std::vector<GraphEntry> graph_cache;
  uint64_t graph_clock = 0;
  // No-allocation mode (t0h_forecast_grouped_dev_noalloc): while `on`, every
  // buffer is carved from the device scratch `dev` and every upload is staged
  // through the pinned `host` region the model allocated at load.
  struct Arena {
    bool on = false;
    uint8_t* dev = nullptr;
    size_t dev_cap = 0, dev_used = 0;
    uint8_t* host = nullptr;
    size_t host_cap = 0, host_used = 0;
    std::unordered_map<std::string, std::pair<void*, size_t>> named;
  } arena;
};

// Per-kernel-kind timing with HIP events recorded on the model's stream around
// each launch of the forward (enabled on demand; off by default).
struct ProfEntry {
  std::string name;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
  uint64_t launches = 0;
  double total_ms = 0.0;
};
struct Profiler {
  bool on = false;
  std::string only;  // when non-empty, only launches of this kind are timed
  std::vector<ProfEntry> entries;
  std::vector<hipEvent_t> spare;
};

}  // namespace t0h

struct t0h_ctx {
  int device = 0;
  std::string arch;
};

struct t0h_model {
  t0h_ctx* ctx = nullptr;
  t0h::ModelConfig mc;
  hipStream_t stream = nullptr;
  uint8_t* d_weights = nullptr;
  size_t weights_bytes = 0;
  uint64_t quantizable_bytes = 0;
  t0h::RBlock enc, dec;
  const float* type_emb = nullptr;
  int n_types = 0;
  const float* out_norm = nullptr;
  std::vector<t0h::Layer> layers;
  t0h::Workspace ws;
  t0h::Profiler prof;
  // pinned host staging of the no-allocation entry point (allocated at load) and
  // the event marking when the last call's copies out of it have executed
  void* noalloc_host = nullptr;
  size_t noalloc_host_bytes = 0;
  hipEvent_t noalloc_ev = nullptr;
  bool noalloc_pending = false;
  // Set to 1 by the device when a forecast's quantile logits are not finite (an
  // f16 activation beyond +-65504 became inf, or the weights hold inf/NaN): an
  // int in coherent pinned host memory (allocated at load), written by the kernel
  // through its device address and read by the host after the stream drains.
  // `nonfinite_unread`: a device-output call may have set it since it was read.
  int* h_nonfinite = nullptr;
  int* d_nonfinite = nullptr;
  bool nonfinite_unread = false;
};

namespace t0h {
namespace {

// ---- workspace (grow-only, like pool.rs:75-93) ----
// No-allocation mode: a named slice of the device scratch (256-byte aligned),
// the same slice for every request of one name within a call.
void* arena_get(t0h_model* m, const char* name, size_t bytes) {
  Workspace::Arena& a = m->ws.arena;
  auto it = a.named.find(name);
  if (it != a.named.end()) {
    if (it->second.second < bytes) throw Error(T0H_ERR_HIP, std::string("internal: scratch slice ") + name + " regrown");
    return it->second.first;
  }
  const size_t off = (a.dev_used + 255) & ~size_t(255);
  if (off + bytes > a.dev_cap)
    throw Error(T0H_ERR_UNSUPPORTED, "window needs more than the " + std::to_string(a.dev_cap >> 20) +
                                         " MiB no-allocation scratch (exhausted at buffer " + name + ", " +
                                         std::to_string(off + bytes) + " bytes so far)");
  a.dev_used = off + bytes;
  void* p = a.dev + off;
  a.named.emplace(name, std::make_pair(p, bytes));
  return p;
}

template <typename T>
T* ws_get(t0h_model* m, const char* name, size_t count) {
  if (m->ws.arena.on) return static_cast<T*>(arena_get(m, name, std::max<size_t>(count * sizeof(T), 256)));
  Buf& b = m->ws.bufs[name];
  const size_t bytes = std::max<size_t>(count * sizeof(T), 256);
  if (b.cap < bytes) {
    if (m->ws.capturing)
      throw Error(T0H_ERR_HIP, std::string("internal: workspace buffer ") + name + " grew during graph capture");
    if (b.p) {
      hip_check(hipStreamSynchronize(m->stream), "hipStreamSynchronize");
      hip_check(hipFree(b.p), "hipFree");
      b.p = nullptr;
      b.cap = 0;
    }
    const size_t want = bytes + bytes / 4;
    if (hipMalloc(&b.p, want) != hipSuccess) {
      (void)hipGetLastError();
      throw Error(T0H_ERR_OOM, std::string("device allocation of ") + std::to_string(want) + " bytes failed (" + name + ")");
    }
    b.cap = want;
    m->ws.allocs++;
  }
  return static_cast<T*>(b.p);
}

// Copy n host elements into device buffer `name` (grown as needed), stream-ordered.
// The host data is first copied into a pinned staging buffer owned by the model, so
// the caller's memory may be released as soon as this returns.
template <typename T>
T* put(t0h_model* m, const char* name, const T* src, size_t n) {
  T* dst = ws_get<T>(m, name, n);
  if (n == 0) return dst;
  const size_t bytes = n * sizeof(T);
  if (m->ws.arena.on) {  // staged through the pinned region allocated at load
    Workspace::Arena& a = m->ws.arena;
    const size_t off = (a.host_used + 63) & ~size_t(63);
    if (off + bytes > a.host_cap)
      throw Error(T0H_ERR_UNSUPPORTED, std::string("no-allocation host staging exhausted at ") + name);
    a.host_used = off + bytes;
    std::memcpy(a.host + off, src, bytes);
    hip_check(hipMemcpyAsync(dst, a.host + off, bytes, hipMemcpyHostToDevice, m->stream), "hipMemcpyAsync H2D");
    return dst;
  }
  Stage& st = m->ws.stages[name];
  if (st.pending) {
    hip_check(hipEventSynchronize(st.ev), "hipEventSynchronize");
    st.pending = false;
  }
  if (!st.ev) hip_check(hipEventCreateWithFlags(&st.ev, hipEventDisableTiming), "hipEventCreate");
  if (st.cap < bytes) {
    if (st.p) hip_check(hipHostFree(st.p), "hipHostFree");
    st.p = nullptr;
    st.cap = 0;
    if (hipHostMalloc(&st.p, bytes + bytes / 4, hipHostMallocDefault) != hipSuccess) {
      (void)hipGetLastError();
      throw Error(T0H_ERR_OOM, "pinned host allocation failed");
    }
    st.cap = bytes + bytes / 4;
  }
  std::memcpy(st.p, src, bytes);
  hip_check(hipMemcpyAsync(dst, st.p, bytes, hipMemcpyHostToDevice, m->stream), "hipMemcpyAsync H2D");
  hip_check(hipEventRecord(st.ev, m->stream), "hipEventRecord");
  st.pending = true;
  return dst;
}
// put() for small metadata arrays that often repeat call to call: skipped when
// the bytes equal the last ones this buffer received through put_cached and
// the buffer has not been reallocated since (nothing else writes these buffers).
template <typename T>
const T* put_cached(t0h_model* m, const char* name, const T* src, size_t n) {
  if (m->ws.arena.on) return put(m, name, src, n);  // the scratch keeps no contents of its own
  const size_t bytes = n * sizeof(T);
  const uint64_t gen = m->ws.allocs;
  T* dst = ws_get<T>(m, name, n);
  std::vector<uint8_t>& sh = m->ws.shadow[name];
  const bool same = gen == m->ws.allocs && sh.size() == bytes + sizeof(void*) &&
                    std::memcmp(sh.data(), &dst, sizeof(void*)) == 0 &&
                    (bytes == 0 || std::memcmp(sh.data() + sizeof(void*), src, bytes) == 0);
  if (same) return dst;
  put(m, name, src, n);
  sh.resize(bytes + sizeof(void*));
  std::memcpy(sh.data(), &dst, sizeof(void*));
  if (bytes) std::memcpy(sh.data() + sizeof(void*), src, bytes);
  return dst;
}

template <typename T>
void download(t0h_model* m, T* dst, const T* src, size_t n) {
  if (n) hip_check(hipMemcpyAsync(dst, src, n * sizeof(T), hipMemcpyDeviceToHost, m->stream), "hipMemcpyAsync D2H");
}
void sync(t0h_model* m) { hip_check(hipStreamSynchronize(m->stream), "hipStreamSynchronize"); }

hipEvent_t prof_event(t0h_model* m) {
  if (!m->prof.spare.empty()) {
    hipEvent_t e = m->prof.spare.back();
    m->prof.spare.pop_back();
    return e;
  }
  hipEvent_t e;
  hip_check(hipEventCreate(&e), "hipEventCreate");
  return e;
}

// Scope guard: times the launches issued inside it under `name`.
struct ProfScope {
  t0h_model* m;
  size_t idx = 0;
  hipEvent_t start = nullptr;
  ProfScope(t0h_model* model, const char* name) : m(model) {
    if (!m->prof.on) return;
    if (!m->prof.only.empty() && m->prof.only != name) return;
    auto& es = m->prof.entries;
    idx = es.size();
    for (size_t i = 0; i < es.size(); ++i)
      if (es[i].name == name) idx = i;
    if (idx == es.size()) {
      es.emplace_back();
      es.back().name = name;
    }
    start = prof_event(m);
    hip_check(hipEventRecord(start, m->stream), "hipEventRecord");
  }
  ~ProfScope() {
    if (!start) return;
    hipEvent_t end = prof_event(m);
    if (hipEventRecord(end, m->stream) == hipSuccess) m->prof.entries[idx].pending.emplace_back(start, end);
  }
};

void prof_collect(t0h_model* m) {
  bool any = false;
  for (auto& e : m->prof.entries) any |= !e.pending.empty();
  if (!any) return;
  sync(m);
  for (auto& e : m->prof.entries) {
    for (auto& pr : e.pending) {
      float ms = 0.0f;
      hip_check(hipEventElapsedTime(&ms, pr.first, pr.second), "hipEventElapsedTime");
      e.total_ms += ms;
      e.launches++;
      m->prof.spare.push_back(pr.first);
      m->prof.spare.push_back(pr.second);
    }
    e.pending.clear();
  }
}

// ---- load ----
size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct Placement {
  const GgufTensor* t;
  bool as_matrix;  // device keeps GGUF blocks/f16 rows; else f32 vector
  int dev_type;
  size_t off, bytes;
};

void load_model(t0h_model* m, const uint8_t* bytes, size_t len) {
  GgufFile f = read_gguf(bytes, len);
  m->mc = config_from_meta(f);
  const t0h_config& c = m->mc.c;
  validate_model(f, c);
  if (c.embed_dim / c.num_heads != 64)
    throw Error(T0H_ERR_UNSUPPORTED, "this engine's attention kernels require head_dim 64");
  if (c.embed_dim % 64 || c.mlp_hidden_dim % 64 || (3 * c.patch_size) % 32)
    throw Error(T0H_ERR_UNSUPPORTED, "embed_dim and mlp_hidden_dim must be multiples of 64 and 3*patch_size of 32");

  std::vector<std::string> matrices = {"patch_encoder.projection.mlp.hidden_layer.weight",
                                       "patch_encoder.projection.mlp.output_layer.weight",
                                       "patch_encoder.projection.residual_layer.weight",
                                       "decoder.mlp.hidden_layer.weight",
                                       "decoder.mlp.output_layer.weight",
                                       "decoder.residual_layer.weight"};
  std::vector<std::string> vectors = {"patch_encoder.projection.mlp.hidden_layer.bias",
                                      "patch_encoder.projection.mlp.output_layer.bias",
                                      "patch_encoder.projection.residual_layer.bias",
                                      "patch_encoder.type_embeddings.weight",
                                      "transformer.out_norm.scale",
                                      "decoder.mlp.hidden_layer.bias",
                                      "decoder.mlp.output_layer.bias",
                                      "decoder.residual_layer.bias"};
  const std::vector<bool> types = layer_types(c);
  for (size_t i = 0; i < types.size(); ++i) {
    const std::string p = "transformer.layers." + std::to_string(i);
    for (const char* s : {".attention_block.attention.wQKV.weight", ".attention_block.attention.wO.weight",
                          ".mlp.0.weight", ".mlp.2.weight"})
      matrices.push_back(p + s);
    for (const char* s : {".attention_block.norm.scale", ".attention_block.attention.wQKV.bias",
                          ".attention_block.attention.wO.bias", ".attention_block.attention.q_norm.scale",
                          ".attention_block.attention.k_norm.scale", ".norm.scale", ".mlp.0.bias", ".mlp.2.bias"})
      vectors.push_back(p + s);
  }
  std::unordered_map<std::string, Placement> place;
  size_t off = 0;
  for (const auto& n : matrices) {
    const GgufTensor& t = f.tensors.at(n);
    Placement pl{&t, true, t.type == T0H_F32 ? T0H_F16 : t.type, off, 0};
    pl.bytes = t.type == T0H_F32 ? t.n * 2 : t.nbytes;
    off = align256(off + pl.bytes);
    place[n] = pl;
  }
  for (const auto& n : vectors) {
    const GgufTensor& t = f.tensors.at(n);
    Placement pl{&t, false, T0H_F32, off, t.n * 4};
    off = align256(off + pl.bytes);
    place[n] = pl;
  }
  std::vector<uint8_t> host(off, 0);
  for (auto& kv : place) {
    const Placement& pl = kv.second;
    uint8_t* dst = host.data() + pl.off;
    if (!pl.as_matrix) {
      dequantize(pl.t->type, pl.t->data, pl.t->n, reinterpret_cast<float*>(dst));
    } else if (pl.t->type == T0H_F32) {  // f32 matrices are held as f16 rows
      std::vector<float> tmp(pl.t->n);
      std::memcpy(tmp.data(), pl.t->data, pl.t->n * 4);
      quantize(T0H_F16, tmp.data(), tmp.size(), dst);
    } else {
      std::memcpy(dst, pl.t->data, pl.t->nbytes);  // GGUF blocks verbatim
    }
  }
  if (hipMalloc(&m->d_weights, off) != hipSuccess) {
    (void)hipGetLastError();
    throw Error(T0H_ERR_OOM, "device allocation for weights failed");
  }
  m->weights_bytes = off;
  hip_check(hipMemcpy(m->d_weights, host.data(), off, hipMemcpyHostToDevice), "hipMemcpy weights");

  auto mat = [&](const std::string& n) {
    const Placement& pl = place.at(n);
    Mat x;
    x.w = m->d_weights + pl.off;
    x.type = pl.dev_type;
    x.n = (int)pl.t->shape[0];
    x.k = (int)pl.t->shape[1];
    x.bytes = pl.bytes;
    return x;
  };
  auto vec = [&](const std::string& n) { return reinterpret_cast<const float*>(m->d_weights + place.at(n).off); };
  auto rblock = [&](const std::string& p) {
    RBlock b;
    b.hid = mat(p + ".mlp.hidden_layer.weight");
    b.out = mat(p + ".mlp.output_layer.weight");
    b.res = mat(p + ".residual_layer.weight");
    b.hb = vec(p + ".mlp.hidden_layer.bias");
    b.ob = vec(p + ".mlp.output_layer.bias");
    b.rb = vec(p + ".residual_layer.bias");
    return b;
  };
  m->enc = rblock("patch_encoder.projection");
  m->dec = rblock("decoder");
  if (m->enc.hid.n % 64 || m->dec.hid.n % 64)
    throw Error(T0H_ERR_UNSUPPORTED, "residual-block hidden widths must be multiples of 64");
  m->type_emb = vec("patch_encoder.type_embeddings.weight");
  m->n_types = (int)f.tensors.at("patch_encoder.type_embeddings.weight").shape[0];
  m->out_norm = vec("transformer.out_norm.scale");
  m->quantizable_bytes = 0;
  for (size_t i = 0; i < types.size(); ++i) {
    const std::string p = "transformer.layers." + std::to_string(i);
    Layer L;
    L.group = types[i];
    L.qkv = mat(p + ".attention_block.attention.wQKV.weight");
    L.o = mat(p + ".attention_block.attention.wO.weight");
    L.w0 = mat(p + ".mlp.0.weight");
    L.w2 = mat(p + ".mlp.2.weight");
    L.b_qkv = vec(p + ".attention_block.attention.wQKV.bias");
    L.b_o = vec(p + ".attention_block.attention.wO.bias");
    L.b0 = vec(p + ".mlp.0.bias");
    L.b2 = vec(p + ".mlp.2.bias");
    L.norm = vec(p + ".attention_block.norm.scale");
    L.mlp_norm = vec(p + ".norm.scale");
    L.q_norm = vec(p + ".attention_block.attention.q_norm.scale");
    L.k_norm = vec(p + ".attention_block.attention.k_norm.scale");
    auto host_vec = [&](const std::string& n) {
      const float* f = reinterpret_cast<const float*>(host.data() + place.at(n).off);
      return std::vector<float>(f, f + place.at(n).t->n);
    };
    L.q_norm_h = host_vec(p + ".attention_block.attention.q_norm.scale");
    L.k_norm_h = host_vec(p + ".attention_block.attention.k_norm.scale");
    m->quantizable_bytes += L.qkv.bytes + L.o.bytes + L.w0.bytes + L.w2.bytes;
    m->layers.push_back(L);
  }
}

// ---- RoPE tables (ops.rs:77-116): f64 math, f32 tables, xpos halves-concat ----
void rope_tables(int p, int hd, std::vector<float>& cs, std::vector<float>& sn, std::vector<float>& sc) {
  cs.assign((size_t)p * hd, 0.f);
  sn.assign((size_t)p * hd, 0.f);
  sc.assign((size_t)p * hd, 0.f);
  const int half = hd / 2;
  const double theta = 10000.0, scale_base = 512.0;
  const double max_half = std::floor((double)(p - 1) / 2.0);
  for (int pos = 0; pos < p; ++pos) {
    const double power = ((double)pos - max_half) / scale_base;
    for (int j = 0; j < half; ++j) {
      const double inv_freq = 1.0 / std::pow(theta, (double)(2 * j) / (double)hd);
      const double angle = (double)pos * inv_freq;
      const double base = (2.0 * j + 0.4 * hd) / (1.4 * hd);
      const float s = (float)std::pow(base, power);
      for (int k = 0; k < 2; ++k) {
        cs[(size_t)pos * hd + 2 * j + k] = (float)std::cos(angle);
        sn[(size_t)pos * hd + 2 * j + k] = (float)std::sin(angle);
      }
      sc[(size_t)pos * hd + j] = s;
      sc[(size_t)pos * hd + half + j] = s;
    }
  }
}

// ---- group segments: rows sorted by group; per row its segment -------------
void upload_segments(t0h_model* m, const std::vector<int64_t>& row_group, bool consistent) {
  const int v = (int)row_group.size();
  std::vector<int> perm(v), begin(v), len(v), starts;
  std::iota(perm.begin(), perm.end(), 0);
  if (consistent) {
    std::stable_sort(perm.begin(), perm.end(), [&](int a, int b) { return row_group[a] < row_group[b]; });
    int i = 0;
    while (i < v) {
      int j = i;
      while (j < v && row_group[perm[j]] == row_group[perm[i]]) ++j;
      for (int k = i; k < j; ++k) {
        begin[perm[k]] = i;
        len[perm[k]] = j - i;
      }
      starts.push_back(i);
      i = j;
    }
  } else {  // arbitrary per-patch groups: every row scans all rows (group equality is checked per key)
    std::fill(begin.begin(), begin.end(), 0);
    std::fill(len.begin(), len.end(), v);
    if (v) starts.push_back(0);
  }
  put_cached(m, "perm", perm.data(), v);
  put_cached(m, "seg_begin", begin.data(), v);
  put_cached(m, "seg_len", len.data(), v);
  ws_get<int>(m, "seg_start", v);  // sized for the most segments, so the count may vary without a regrow
  if (!starts.empty()) put_cached(m, "seg_start", starts.data(), starts.size());
  m->ws.seg_max = v ? *std::max_element(len.begin(), len.end()) : 0;
  m->ws.n_seg = (int)starts.size();
}

// Per layer and side (q, k), one [p, 128] f32 table folding the QK-norm scale,
// the rotation and the xpos scale (q: scale, k: scale.recip() in f32) of each
// element, so that rotated = inv_rms * (x[e] * A[e] + x[e^1] * B[e]) with
//   A[e] = norm[e] * cos[e] * xs[e]             (columns 0..63)
//   B[e] = -+ norm[e^1] * sin[e] * xs[e]        (columns 64..127; - for even e)
// which is ops.rs:132-142 applied to ops.rs:175-181's normalized rows, with the
// f32 table values multiplied in f64 and rounded once.
void ensure_rope(t0h_model* m, int p) {
  const bool arena = m->ws.arena.on;  // scratch contents are not kept between calls
  if (!arena && m->ws.rope_p == p) return;
  std::vector<float> cs, sn, sc;
  rope_tables(p, 64, cs, sn, sc);
  const size_t per = (size_t)p * 128;
  std::vector<float> t(m->layers.size() * 2 * per, 0.f);
  for (size_t li = 0; li < m->layers.size(); ++li) {
    const Layer& L = m->layers[li];
    for (int side = 0; side < 2; ++side) {
      const std::vector<float>& nrm = side ? L.k_norm_h : L.q_norm_h;
      float* dst = t.data() + (li * 2 + side) * per;
      for (int pos = 0; pos < p; ++pos)
        for (int e = 0; e < 64; ++e) {
          const size_t i = (size_t)pos * 64 + e;
          const double xs = side ? (double)(1.0f / sc[i]) : (double)sc[i];
          dst[(size_t)pos * 128 + e] = (float)((double)nrm[e] * (double)cs[i] * xs);
          dst[(size_t)pos * 128 + 64 + e] = (float)((e & 1 ? 1.0 : -1.0) * (double)nrm[e ^ 1] * (double)sn[i] * xs);
        }
    }
  }
  put(m, "rope", t.data(), t.size());
  if (!arena) m->ws.rope_p = p;
}

GemmDesc gemm(const Mat& w, const void* a, int lda, const float* bias, void* y, int ldy, int M, int epi, int relu = 0) {
  GemmDesc d;
  d.wtype = w.type;
  d.w = w.w;
  d.a = a;
  d.lda = lda;
  d.bias = bias;
  d.y = y;
  d.ldy = ldy;
  d.M = M;
  d.N = epi == EPI_SWIGLU_F16 ? w.n / 2 : w.n;
  d.K = w.k;
  d.relu = relu;
  d.epi = epi;
  return d;
}

struct PatchMeta {
  _Float16* enc_in;
  int *grp, *type_idx, *type_raw;
  uint8_t *att, *fut;
  float *patch_loc, *patch_scale;
};

PatchMeta patch_buffers(t0h_model* m, int v, int p) {
  const size_t M = (size_t)v * p;
  const int ps = (int)m->mc.c.patch_size;
  PatchMeta pm;
  pm.enc_in = ws_get<_Float16>(m, "enc_in", M * 3 * ps);
  pm.grp = ws_get<int>(m, "grp", M);
  pm.type_idx = ws_get<int>(m, "type_idx", M);
  pm.type_raw = ws_get<int>(m, "type_raw", M);
  pm.att = ws_get<uint8_t>(m, "att", M);
  pm.fut = ws_get<uint8_t>(m, "fut", v);
  pm.patch_loc = ws_get<float>(m, "patch_loc", M);
  pm.patch_scale = ws_get<float>(m, "patch_scale", M);
  return pm;
}

// Patch encoder + transformer layers (t0-fast model.rs:727-786 ≡ t0-core model.rs:184-229).
// Expects enc_in / patch metadata / segments and the RoPE tables of p patches
// (ensure_rope) in the workspace.  Leaves the f32 residual stream in "x".
// Windows of any patch count are taken (t0-core has no limit); the row count is
// bounded so that every per-row offset of the forward fits the kernels' indexing.
void check_window_rows(int v, int p) {
  if ((int64_t)v * p > (int64_t)1 << 24)
    throw Error(T0H_ERR_UNSUPPORTED, "window of " + std::to_string((int64_t)v * p) + " patch rows exceeds 16M");
}

void encode_and_layers(t0h_model* m, int v, int p, const PatchMeta& pm, float* trace_pe, float* trace_l0) {
  const t0h_config& c = m->mc.c;
  const int E = (int)c.embed_dim, ps = (int)c.patch_size, M = v * p;
  const int H = (int)c.mlp_hidden_dim;
  hipStream_t s = m->stream;
  const int wide = std::max(E, m->enc.hid.n);
  float* x = ws_get<float>(m, "x", (size_t)M * E);
  _Float16* xn = ws_get<_Float16>(m, "xn", (size_t)M * wide);
  _Float16* qkv = ws_get<_Float16>(m, "qkv", (size_t)M * 3 * E);
  _Float16* hb = ws_get<_Float16>(m, "h", (size_t)M * H);
  const int* perm = ws_get<int>(m, "perm", v);
  const int* seg_begin = ws_get<int>(m, "seg_begin", v);
  const int* seg_len = ws_get<int>(m, "seg_len", v);
  const int* seg_start = ws_get<int>(m, "seg_start", v);
  if (!m->ws.arena.on && m->ws.rope_p != p) throw Error(T0H_ERR_HIP, "internal: RoPE tables not prepared for this window");

  // RMSNorm split across the GEMMs either side of it (ops.rs:12-17): each residual
  // GEMM of the layers (wO, w2) also writes f16(x * g / 16) and per-row
  // partial sums of squares, and the consuming GEMM (QKV, SwiGLU) scales its output
  // rows by 16 / sqrt(mean + eps); the patch encoder's output GEMM produces layer 0's.
  // Used below 1024 rows when every kernel involved supports it (one series,
  // config 3: 0.597 -> 0.582 ms: 23 fewer launches); at
  // config 4 it measured 5 % slower (the producers' epilogues +40 us, the consumers'
  // per-tile wait for their rows' sums +24 us, against 68 us of norm launches per
  // layer), so larger windows keep each norm as its own launch.
  _Float16* xnorm = nullptr;
  float* ssq = nullptr;
  bool split = false;
  if (!m->layers.empty() && M < 1024) {
    const Layer& L0 = m->layers[0];
    GemmDesc q = gemm(L0.qkv, xn, E, L0.b_qkv, qkv, 3 * E, M, EPI_STORE_F16);
    GemmDesc w0 = gemm(L0.w0, xn, E, L0.b0, hb, H, M, EPI_SWIGLU_F16);
    GemmDesc res = gemm(L0.o, xn, E, L0.b_o, x, E, M, EPI_RESID_F32);
    GemmDesc res2 = gemm(L0.w2, hb, H, L0.b2, x, E, M, EPI_RESID_F32);
    q.ssq_parts = w0.ssq_parts = E / 32;
    split = rownorm_consumer_ok(q) && rownorm_consumer_ok(w0) && rownorm_producer_ok(res) &&
            rownorm_producer_ok(res2);
    for (size_t li = 1; li < m->layers.size() && split; ++li)  // every layer's weights alike
      split = m->layers[li].qkv.type == L0.qkv.type && m->layers[li].w0.type == L0.w0.type;
  }
  if (split) {
    xnorm = ws_get<_Float16>(m, "xnorm", (size_t)M * E);
    ssq = ws_get<float>(m, "ssq", (size_t)M * (E / 32));
  }
  auto produce = [&](GemmDesc& g, const float* scale) {  // the next norm, into xnorm / ssq
    if (!split || !scale) return;
    g.norm_g = scale;
    g.norm_out = xnorm;
    g.norm_ssq = ssq;
  };
  auto consume = [&](GemmDesc& g) {
    if (!split) return;
    g.a = xnorm;
    g.lda = E;
    g.row_ssq = ssq;
    g.ssq_parts = E / 32;
    g.ssq_dim = E;
  };

  // patch encoder residual block + type embedding (model.rs:199-207); its output
  // GEMM produces layer 0's norm when it can
  bool enc_produces = false;
  {
    ProfScope ps_(m, "gemm_encoder");
    launch_gemm(gemm(m->enc.hid, pm.enc_in, 3 * ps, m->enc.hb, xn, m->enc.hid.n, M, EPI_STORE_F16, 1), s);
    GemmDesc rd = gemm(m->enc.res, pm.enc_in, 3 * ps, m->enc.rb, x, E, M, EPI_STORE_F32);
    rd.row_add = m->type_emb;
    rd.row_add_idx = pm.type_idx;
    launch_gemm(rd, s);
    GemmDesc eo = gemm(m->enc.out, xn, m->enc.hid.n, m->enc.ob, x, E, M, EPI_RESID_F32);
    enc_produces = split && rownorm_producer_ok(eo);
    if (enc_produces) produce(eo, m->layers[0].norm);
    launch_gemm(eo, s);
  }
  if (trace_pe) download(m, trace_pe, x, (size_t)M * E);

  AttnDesc ad;
  ad.qkv = qkv;
  ad.out = xn;
  ad.v = v;
  ad.p = p;
  ad.E = E;
  ad.heads = (int)c.num_heads;
  const float* rope = ws_get<float>(m, "rope", m->layers.size() * 2 * (size_t)p * 128);
  ad.grp = pm.grp;
  ad.att = pm.att;
  ad.fut = pm.fut;
  ad.perm = perm;
  ad.seg_begin = seg_begin;
  ad.seg_len = seg_len;
  ad.seg_max = m->ws.seg_max;
  ad.seg_start = seg_start;
  ad.n_seg = m->ws.n_seg;
  if (p > T0H_LDS_PATCHES) {  // the long-window time attention's key workspace
    const size_t P32 = (size_t)(p + 31) / 32 * 32;
    ad.kr = ws_get<_Float16>(m, "attn_kr", (size_t)v * P32 * E);
    ad.vt = ws_get<_Float16>(m, "attn_vt", (size_t)v * P32 * E);
    ad.kg = ws_get<int>(m, "attn_kg", (size_t)v * P32);
  }
  for (size_t li = 0; li < m->layers.size(); ++li) {
    const Layer& L = m->layers[li];
    if (!split || (li == 0 && !enc_produces)) {
      ProfScope ps_(m, "rmsnorm");
      launch_rmsnorm(x, L.norm, xn, RowGather{}, M, E, s);
    }
    {
      ProfScope ps_(m, "gemm_qkv");
      GemmDesc g = gemm(L.qkv, xn, E, L.b_qkv, qkv, 3 * E, M, EPI_STORE_F16);
      if (li > 0 || enc_produces) consume(g);
      launch_gemm(g, s);
    }
    ad.q_norm = L.q_norm;
    ad.k_norm = L.k_norm;
    ad.rope_q = rope + li * 2 * (size_t)p * 128;
    ad.rope_k = ad.rope_q + (size_t)p * 128;
    // One variate row: every query of a group layer has one key, itself (or,
    // an all-PAD patch, uniform weights over the one row), so the attention
    // output is the value row exactly and wO reads V in place.
    const bool v_in_place = L.group && v == 1;
    if (L.group && !v_in_place) {
      ProfScope ps_(m, "attn_group");
      launch_group_attention(ad, s);
    } else if (!L.group) {
      ProfScope ps_(m, "attn_time");
      launch_time_attention(ad, s);
    }
    {
      ProfScope ps_(m, "gemm_wo_resid");
      GemmDesc g = v_in_place ? gemm(L.o, qkv + 2 * E, 3 * E, L.b_o, x, E, M, EPI_RESID_F32)
                              : gemm(L.o, xn, E, L.b_o, x, E, M, EPI_RESID_F32);
      produce(g, L.mlp_norm);
      launch_gemm(g, s);
    }
    if (!split) {
      ProfScope ps_(m, "rmsnorm");
      launch_rmsnorm(x, L.mlp_norm, xn, RowGather{}, M, E, s);
    }
    {
      ProfScope ps_(m, "gemm_w0_swiglu");
      GemmDesc g = gemm(L.w0, xn, E, L.b0, hb, H, M, EPI_SWIGLU_F16);
      consume(g);
      launch_gemm(g, s);
    }
    {
      ProfScope ps_(m, "gemm_w2_resid");
      GemmDesc g = gemm(L.w2, hb, H, L.b2, x, E, M, EPI_RESID_F32);
      produce(g, li + 1 < m->layers.size() ? m->layers[li + 1].norm : nullptr);  // out_norm stays a launch
      launch_gemm(g, s);
    }
    if (li == 0 && trace_l0) download(m, trace_l0, x, (size_t)M * E);
  }
}

// out_norm + decoder residual block on `rows` rows of x (gathered per `gth`, or all).
float* decode_rows(t0h_model* m, int rows, const RowGather& gth) {
  const t0h_config& c = m->mc.c;
  const int E = (int)c.embed_dim, nout = m->dec.out.n;
  hipStream_t s = m->stream;
  const float* x = ws_get<float>(m, "x", 1);
  _Float16* din = ws_get<_Float16>(m, "dec_in", (size_t)rows * E);
  _Float16* dh = ws_get<_Float16>(m, "dec_h", (size_t)rows * m->dec.hid.n);
  float* dout = ws_get<float>(m, "dec_out", (size_t)rows * nout);
  ProfScope ps_(m, "decoder");
  launch_rmsnorm(x, m->out_norm, din, gth, rows, E, s);
  launch_gemm(gemm(m->dec.hid, din, E, m->dec.hb, dh, m->dec.hid.n, rows, EPI_STORE_F16, 1), s);
  launch_gemm(gemm(m->dec.res, din, E, m->dec.rb, dout, nout, rows, EPI_STORE_F32), s);
  launch_gemm(gemm(m->dec.out, dh, m->dec.hid.n, m->dec.ob, dout, nout, rows, EPI_RESID_F32), s);
  return dout;
}

// Grows every buffer encode_and_layers and decode_rows use for `rows` patch
// rows and `dec_rows` decoded rows, so that neither allocates once launches start.
void reserve_forward(t0h_model* m, int v, int p, int dec_rows) {
  const t0h_config& c = m->mc.c;
  const size_t M = (size_t)v * p, E = c.embed_dim, wide = std::max<size_t>(E, (size_t)m->enc.hid.n);
  if (p > T0H_LDS_PATCHES) {
    const size_t P32 = (size_t)(p + 31) / 32 * 32;
    ws_get<_Float16>(m, "attn_kr", (size_t)v * P32 * E);
    ws_get<_Float16>(m, "attn_vt", (size_t)v * P32 * E);
    ws_get<int>(m, "attn_kg", (size_t)v * P32);
  }
  ws_get<float>(m, "x", M * E);
  ws_get<_Float16>(m, "xn", M * wide);
  ws_get<_Float16>(m, "qkv", M * 3 * E);
  ws_get<_Float16>(m, "h", M * c.mlp_hidden_dim);
  ws_get<_Float16>(m, "xnorm", M * E);  // the split RMSNorm's rows and partial sums (if used)
  ws_get<float>(m, "ssq", M * (E / 32));
  ws_get<_Float16>(m, "dec_in", (size_t)dec_rows * E);
  ws_get<_Float16>(m, "dec_h", (size_t)dec_rows * m->dec.hid.n);
  ws_get<float>(m, "dec_out", (size_t)dec_rows * m->dec.out.n);
}

void destroy_graphs(t0h_model* m) {
  for (GraphEntry& e : m->ws.graph_cache)
    if (e.exec) (void)hipGraphExecDestroy(e.exec);
  m->ws.graph_cache.clear();
}

// Runs `launches` on the model's stream.  The first call with a key runs them
// eagerly, the second captures them into a HIP graph and launches it, later
// ones replay the graph.  Eager always while the profiler records events or
// replay is switched off.  At most kGraphs graphs are kept (least recently
// used evicted); entries of an older workspace generation are dropped.
template <typename F>
void run_graphed(t0h_model* m, const GraphKey& key, F&& launches) {
  constexpr size_t kGraphs = 8;
  Workspace& ws = m->ws;
  if (!ws.graphs || m->prof.on || ws.arena.on) {
    launches();
    return;
  }
  auto& cache = ws.graph_cache;
  // a graph may still be executing: the stream drains before one is destroyed
  auto drop = [&](std::vector<GraphEntry>::iterator it) {
    if (it->exec) {
      sync(m);
      (void)hipGraphExecDestroy(it->exec);
    }
    return cache.erase(it);
  };
  for (auto it = cache.begin(); it != cache.end();) it = it->key.ws_gen != key.ws_gen ? drop(it) : it + 1;
  GraphEntry* e = nullptr;
  for (GraphEntry& g : cache)
    if (g.key == key) e = &g;
  if (!e) {
    launches();
    if (cache.size() >= kGraphs) {
      drop(std::min_element(cache.begin(), cache.end(),
                            [](const GraphEntry& a, const GraphEntry& b) { return a.last_use < b.last_use; }));
    }
    cache.push_back(GraphEntry{key, nullptr, ++ws.graph_clock});
    return;
  }
  e->last_use = ++ws.graph_clock;
  if (!e->exec) {
    hip_check(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    ws.capturing = true;
    hipGraph_t g = nullptr;
    try {
      launches();
    } catch (...) {
      ws.capturing = false;
      if (hipStreamEndCapture(m->stream, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
      (void)hipGetLastError();
      throw;
    }
    ws.capturing = false;
    hip_check(hipStreamEndCapture(m->stream, &g), "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    const hipError_t rc = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    hip_check(rc, "hipGraphInstantiate");
    e->exec = exec;
  }
  hip_check(hipGraphLaunch(e->exec, m->stream), "hipGraphLaunch");
}

// ---- forecast window (lib.rs:50-97) on device ----
struct WindowRows {
  int t_ctx = 0, horizon = 0;
  const float* d_ctx = nullptr;      // device
  std::vector<int64_t> src_off;      // per row, into d_ctx
  std::vector<int> len;              // per row
  std::vector<int64_t> group;        // per row (>= 0)
};

void forecast_window(t0h_model* m, const WindowRows& wr, float* d_out) {
  const t0h_config& c = m->mc.c;
  const int ps = (int)c.patch_size, nq = (int)c.n_quantiles;
  const int v = (int)wr.src_off.size();
  if (v == 0) return;
  if (wr.t_ctx <= 0) throw Error(T0H_ERR_INVALID_ARG, "forecast: context length must be positive");
  const int pad_left = (ps - wr.t_ctx % ps) % ps;
  const int padded_h = (wr.horizon + ps - 1) / ps * ps;
  if (padded_h > T0H_MAX_HORIZON)
    throw Error(T0H_ERR_HORIZON, "single-window forecast can't exceed max_horizon (1024) in one pass -- use forecast_rollout");
  const int t = pad_left + wr.t_ctx + padded_h;
  const int p = t / ps, ctx_p = (wr.t_ctx + pad_left) / ps, hp = padded_h / ps;
  if (m->ws.arena.on && p > T0H_NOALLOC_MAX_PATCHES)
    throw Error(T0H_ERR_UNSUPPORTED, "no-allocation forecast: window of " + std::to_string(p) + " patches exceeds " +
                                         std::to_string(T0H_NOALLOC_MAX_PATCHES));
  check_window_rows(v, p);
  hipStream_t s = m->stream;

  // dense group ids for the device
  std::vector<int64_t> sorted(wr.group);
  std::sort(sorted.begin(), sorted.end());
  sorted.erase(std::unique(sorted.begin(), sorted.end()), sorted.end());
  std::vector<int> dense(v);
  std::vector<int64_t> dense64(v);
  for (int r = 0; r < v; ++r) {
    dense[r] = (int)(std::lower_bound(sorted.begin(), sorted.end(), wr.group[r]) - sorted.begin());
    dense64[r] = dense[r];
  }
  // every device buffer of the window is sized before the first upload or launch
  const PatchMeta pm = patch_buffers(m, v, p);
  reserve_forward(m, v, p, v * std::max(hp, 1));
  ws_get<int64_t>(m, "win_off", v);
  for (const char* n : {"win_len", "win_grp", "perm", "seg_begin", "seg_len", "seg_start"}) ws_get<int>(m, n, v);
  ws_get<float>(m, "rope", m->layers.size() * 2 * (size_t)p * 128);
  uint8_t* prep_rows = prep_fits_lds(t, ps) ? nullptr : ws_get<uint8_t>(m, "prep_rows", (size_t)v * prep_row_bytes(t, ps));

  const int64_t* d_off = put_cached(m, "win_off", wr.src_off.data(), v);
  const int* d_len = put_cached(m, "win_len", wr.len.data(), v);
  const int* d_grp = put_cached(m, "win_grp", dense.data(), v);
  upload_segments(m, dense64, true);
  ensure_rope(m, p);

  WindowDesc w;
  w.ctx = wr.d_ctx;
  w.src_off = d_off;
  w.len = d_len;
  w.group = d_grp;
  w.v = v;
  w.t_ctx = wr.t_ctx;
  w.horizon = wr.horizon;
  w.pad_left = pad_left;
  w.t = t;
  w.ps = ps;
  w.use_arcsinh = c.scaler_use_arcsinh;
  w.variance_offset = c.scaler_variance_offset;
  w.eps = c.scaler_eps;
  w.rows_mem = prep_rows;

  auto launches = [&]() {
    {
      ProfScope ps_(m, "prep");
      PatchOut po{pm.enc_in, pm.grp, pm.att, pm.type_idx, pm.type_raw, pm.fut, pm.patch_loc, pm.patch_scale};
      launch_window_prep(w, po, s);
    }
    encode_and_layers(m, v, p, pm, nullptr, nullptr);
    if (hp == 0) return;
    float* dout = decode_rows(m, v * hp, RowGather{p, ctx_p, hp});
    ProfScope ps_(m, "forecast_out");
    ForecastOutDesc od;
    od.dec = dout;
    od.patch_loc = pm.patch_loc;
    od.patch_scale = pm.patch_scale;
    od.out = d_out;
    od.nonfinite = m->d_nonfinite;
    od.v = v;
    od.p = p;
    od.ctx_p = ctx_p;
    od.hp = hp;
    od.ps = ps;
    od.nq = nq;
    od.horizon = wr.horizon;
    od.use_arcsinh = c.scaler_use_arcsinh;
    launch_forecast_out(od, s);
  };
  GraphKey key;
  key.v = v;
  key.t_ctx = wr.t_ctx;
  key.horizon = wr.horizon;
  key.seg_max = m->ws.seg_max;
  key.n_seg = m->ws.n_seg;
  key.ctx = wr.d_ctx;
  key.out = d_out;
  key.ws_gen = m->ws.allocs;
  run_graphed(m, key, launches);
}

void require(bool ok, const char* msg) {
  if (!ok) throw Error(T0H_ERR_INVALID_ARG, msg);
}

void bind_device(const t0h_model* m) { hip_check(hipSetDevice(m->ctx->device), "hipSetDevice"); }

float* upload_contexts(t0h_model* m, const float* ctx, size_t n) { return put(m, "ctx_in", ctx, n); }

void check_out(size_t out_len, size_t want) {
  if (out_len != want)
    throw Error(T0H_ERR_INVALID_ARG, "output buffer holds " + std::to_string(out_len) + " floats, expected " + std::to_string(want));
}

// The non-finite flag around a host-output call: if a device-output call may have
// set it, the stream drains and it is cleared before this call's work.
void numerics_begin(t0h_model* m) {
  if (!m->nonfinite_unread) return;
  sync(m);
  *static_cast<volatile int*>(m->h_nonfinite) = 0;
  m->nonfinite_unread = false;
}
// After the stream has drained: raises T0H_ERR_NUMERIC (clearing the flag) if set.
void numerics_end(t0h_model* m) {
  volatile int* f = m->h_nonfinite;
  if (!*f) return;
  *f = 0;
  throw Error(T0H_ERR_NUMERIC,
              "forecast produced non-finite model outputs: an f16 activation exceeded 65504, or the weights are not finite");
}
// A host-output call's end: its n results at d_out come back through pinned
// staging (one asynchronous copy), the stream drains, the numeric flag is checked.
void finish_host_call(t0h_model* m, float* out, const float* d_out, size_t n) {
  const size_t bytes = n * sizeof(float);
  if (bytes) {
    Stage& st = m->ws.stages["results"];
    if (st.cap < bytes) {
      if (st.p) hip_check(hipHostFree(st.p), "hipHostFree");
      st.p = nullptr;
      st.cap = 0;
      if (hipHostMalloc(&st.p, bytes + bytes / 4, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        throw Error(T0H_ERR_OOM, "pinned host allocation failed");
      }
      st.cap = bytes + bytes / 4;
    }
    hip_check(hipMemcpyAsync(st.p, d_out, bytes, hipMemcpyDeviceToHost, m->stream), "hipMemcpyAsync D2H");
    sync(m);
    std::memcpy(out, st.p, bytes);
  } else {
    sync(m);
  }
  numerics_end(m);
}

// forecast_rollout helpers (quantile.rs:16-76)
std::vector<float> interpolate_quantiles(const std::vector<float>& query, const float* levels_in, const float* values_in,
                                         size_t nl) {
  std::vector<size_t> idx(nl);
  std::iota(idx.begin(), idx.end(), 0);
  std::stable_sort(idx.begin(), idx.end(), [&](size_t a, size_t b) { return levels_in[a] < levels_in[b]; });
  std::vector<float> lv, vv;
  for (size_t i : idx) {
    lv.push_back(levels_in[i]);
    vv.push_back(values_in[i]);
  }
  if (lv.front() > 0.0f) {
    lv.insert(lv.begin(), 0.0f);
    vv.insert(vv.begin(), vv.front());
  }
  if (lv.back() < 1.0f) {
    lv.push_back(1.0f);
    vv.push_back(vv.back());
  }
  std::vector<float> out;
  for (float q : query) {
    size_t upper = std::upper_bound(lv.begin(), lv.end(), q) - lv.begin();  // partition_point(l <= q)
    upper = std::min(upper, lv.size() - 1);
    size_t lower = upper > 0 ? upper - 1 : 0;
    const float diff = lv[upper] - lv[lower];
    const float wt = diff == 0.0f ? 0.0f : (q - lv[lower]) / diff;
    out.push_back(vv[lower] + wt * (vv[upper] - vv[lower]));
  }
  return out;
}
std::vector<float> weighted_quantile(const std::vector<float>& query, const std::vector<float>& weights,
                                     const std::vector<float>& samples) {
  float sum = 0.0f;
  for (float w : weights) sum += w;
  std::vector<size_t> idx(samples.size());
  std::iota(idx.begin(), idx.end(), 0);
  std::stable_sort(idx.begin(), idx.end(), [&](size_t a, size_t b) { return samples[a] < samples[b]; });
  std::vector<float> ss, cw;
  float cum = 0.0f;
  for (size_t i : idx) {
    ss.push_back(samples[i]);
    cum += weights[i] / sum;
    cw.push_back(std::min(1.0f, std::max(0.0f, cum)));
  }
  return interpolate_quantiles(query, cw.data(), ss.data(), ss.size());
}
std::vector<float> prob_mass(const float* levels, size_t n) {
  std::vector<float> b(n + 2);
  b[0] = 0.0f;
  std::copy(levels, levels + n, b.begin() + 1);
  b[n + 1] = 1.0f;
  std::vector<float> mass(n);
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    mass[i] = (b[i + 2] - b[i]) / 2.0f;
    sum += mass[i];
  }
  for (float& x : mass) x /= sum;
  return mass;
}

int median_index(const t0h_config& c) {
  int best = 0;
  for (int i = 1; i < (int)c.n_quantiles; ++i)
    if (std::fabs(c.quantile_levels[i] - 0.5f) < std::fabs(c.quantile_levels[best] - 0.5f)) best = i;
  return best;
}

}  // namespace

// Exposed for the rollout driver.
void forecast_host(t0h_model* m, const float* ctx, size_t v, size_t t_ctx, size_t horizon, float* out) {
  const int nq = (int)m->mc.c.n_quantiles;
  numerics_begin(m);
  float* d_ctx = upload_contexts(m, ctx, v * t_ctx);
  WindowRows wr;
  wr.t_ctx = (int)t_ctx;
  wr.horizon = (int)horizon;
  wr.d_ctx = d_ctx;
  for (size_t r = 0; r < v; ++r) {
    wr.src_off.push_back((int64_t)(r * t_ctx));
    wr.len.push_back((int)t_ctx);
    wr.group.push_back(0);  // data.rs:57 one shared group id
  }
  float* d_out = ws_get<float>(m, "out", std::max<size_t>(1, v * horizon * nq));
  forecast_window(m, wr, d_out);
  finish_host_call(m, out, d_out, v * horizon * nq);
}

void forecast_batch_host(t0h_model* m, const float* ctx, size_t n, size_t t_ctx, size_t horizon, size_t chunk,
                         float* out) {
  const int nq = (int)m->mc.c.n_quantiles;
  chunk = (chunk == 0 || chunk > n) ? n : chunk;
  numerics_begin(m);
  float* d_ctx = upload_contexts(m, ctx, n * t_ctx);
  float* d_out = ws_get<float>(m, "out", std::max<size_t>(1, n * horizon * nq));
  for (size_t start = 0; start < n; start += chunk) {
    const size_t k = std::min(chunk, n - start);
    WindowRows wr;
    wr.t_ctx = (int)t_ctx;
    wr.horizon = (int)horizon;
    wr.d_ctx = d_ctx;
    for (size_t r = 0; r < k; ++r) {
      wr.src_off.push_back((int64_t)((start + r) * t_ctx));
      wr.len.push_back((int)t_ctx);
      wr.group.push_back((int64_t)r);  // data.rs:96-105 distinct group per signal
    }
    forecast_window(m, wr, d_out + start * horizon * nq);
  }
  finish_host_call(m, out, d_out, n * horizon * nq);
}

}  // namespace t0h

using namespace t0h;

#define API_BEGIN try {
#define API_END                                    \
  }                                                \
  catch (const t0h::Error& e) {                    \
    set_error(e.what());                           \
    return e.code;                                 \
  }                                                \
  catch (const std::bad_alloc&) {                  \
    set_error("host allocation failed");           \
    return T0H_ERR_OOM;                            \
  }                                                \
  catch (const std::exception& e) {                \
    set_error(std::string("internal error: ") + e.what()); \
    return T0H_ERR_INVALID_ARG;                    \
  }                                                \
  return T0H_OK;

extern "C" {

const char* t0h_last_error(void) { return g_last_error.c_str(); }
int t0h_abi_version(void) { return T0H_ABI_VERSION; }

int t0h_ctx_create(int device, t0h_ctx** out) {
  API_BEGIN
  require(out != nullptr, "t0h_ctx_create: out is NULL");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
    (void)hipGetLastError();
    throw Error(T0H_ERR_NO_DEVICE, "no GPU device available");
  }
  if (device < 0 || device >= n) throw Error(T0H_ERR_NO_DEVICE, "device index out of range");
  hip_check(hipSetDevice(device), "hipSetDevice");
  hipDeviceProp_t prop;
  hip_check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  std::string arch = prop.gcnArchName;
  if (arch.rfind("gfx950", 0) != 0)
    throw Error(T0H_ERR_UNSUPPORTED, "this library is built for gfx950 (MI355X); device is " + arch);
  scratch_init();  // this device's no-allocation scratch address, once
  auto* c = new t0h_ctx;
  c->device = device;
  c->arch = arch;
  *out = c;
  API_END
}

void t0h_ctx_destroy(t0h_ctx* ctx) { delete ctx; }

int t0h_gguf_inspect(const uint8_t* bytes, size_t len, t0h_config* cfg, size_t* n_tensors) {
  API_BEGIN
  require(bytes != nullptr || len == 0, "t0h_gguf_inspect: bytes is NULL");
  GgufFile f = read_gguf(bytes, len);
  ModelConfig mc = config_from_meta(f);
  validate_model(f, mc.c);
  if (cfg) *cfg = mc.c;
  if (n_tensors) *n_tensors = f.tensors.size();
  API_END
}

int t0h_model_load_gguf(t0h_ctx* ctx, const uint8_t* bytes, size_t len, t0h_model** out) {
  API_BEGIN
  require(ctx && out, "t0h_model_load_gguf: NULL argument");
  require(bytes != nullptr || len == 0, "t0h_model_load_gguf: bytes is NULL");
  *out = nullptr;
  hip_check(hipSetDevice(ctx->device), "hipSetDevice");
  std::unique_ptr<t0h_model> m(new t0h_model);
  m->ctx = ctx;
  hip_check(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking), "hipStreamCreate");
  try {
    load_model(m.get(), bytes, len);
    // pinned staging for the no-allocation entry point: RoPE tables of the longest
    // window plus per-row metadata for as many rows as the scratch can hold
    const size_t rows_max = T0H_NOALLOC_SCRATCH_BYTES / (4 * (size_t)m->mc.c.embed_dim);
    m->noalloc_host_bytes = m->layers.size() * 2 * (size_t)T0H_NOALLOC_MAX_PATCHES * 128 * 4 + 32 * rows_max + 4096;
    if (hipHostMalloc(&m->noalloc_host, m->noalloc_host_bytes, hipHostMallocDefault) != hipSuccess) {
      (void)hipGetLastError();
      m->noalloc_host = nullptr;
      throw Error(T0H_ERR_OOM, "pinned host allocation failed");
    }
    hip_check(hipEventCreateWithFlags(&m->noalloc_ev, hipEventDisableTiming), "hipEventCreate");
    void* flag = nullptr;
    if (hipHostMalloc(&flag, 64, hipHostMallocCoherent) != hipSuccess) {
      (void)hipGetLastError();
      throw Error(T0H_ERR_OOM, "pinned host allocation failed");
    }
    m->h_nonfinite = static_cast<int*>(flag);
    *m->h_nonfinite = 0;
    void* dflag = nullptr;
    hip_check(hipHostGetDevicePointer(&dflag, flag, 0), "hipHostGetDevicePointer");
    m->d_nonfinite = static_cast<int*>(dflag);
  } catch (...) {
    if (m->h_nonfinite) (void)hipHostFree(m->h_nonfinite);
    if (m->noalloc_ev) (void)hipEventDestroy(m->noalloc_ev);
    if (m->noalloc_host) (void)hipHostFree(m->noalloc_host);
    if (m->d_weights) (void)hipFree(m->d_weights);
    (void)hipStreamDestroy(m->stream);
    throw;
  }
  *out = m.release();
  API_END
}

void t0h_model_destroy(t0h_model* m) {
  if (!m) return;
  (void)hipSetDevice(m->ctx->device);
  (void)hipStreamSynchronize(m->stream);
  destroy_graphs(m);
  for (auto& kv : m->ws.bufs)
    if (kv.second.p) (void)hipFree(kv.second.p);
  for (auto& kv : m->ws.stages) {
    if (kv.second.p) (void)hipHostFree(kv.second.p);
    if (kv.second.ev) (void)hipEventDestroy(kv.second.ev);
  }
  for (auto& e : m->prof.entries)
    for (auto& pr : e.pending) {
      (void)hipEventDestroy(pr.first);
      (void)hipEventDestroy(pr.second);
    }
  for (hipEvent_t e : m->prof.spare) (void)hipEventDestroy(e);
  if (m->noalloc_host) (void)hipHostFree(m->noalloc_host);
  if (m->noalloc_ev) (void)hipEventDestroy(m->noalloc_ev);
  if (m->h_nonfinite) (void)hipHostFree(m->h_nonfinite);
  if (m->d_weights) (void)hipFree(m->d_weights);
  (void)hipStreamDestroy(m->stream);
  delete m;
}

int t0h_model_config(const t0h_model* m, t0h_config* out) {
  API_BEGIN
  require(m && out, "t0h_model_config: NULL argument");
  *out = m->mc.c;
  out->num_layers = (uint32_t)m->layers.size();
  API_END
}

int t0h_model_weight_bytes(const t0h_model* m, uint64_t* quantizable, uint64_t* total) {
  API_BEGIN
  require(m != nullptr, "t0h_model_weight_bytes: NULL model");
  if (quantizable) *quantizable = m->quantizable_bytes;
  if (total) *total = m->weights_bytes;
  API_END
}

void* t0h_model_stream(const t0h_model* m) { return m ? (void*)m->stream : nullptr; }

int t0h_model_workspace(const t0h_model* m, uint64_t* resident, uint64_t* allocs) {
  API_BEGIN
  require(m != nullptr, "t0h_model_workspace: NULL model");
  uint64_t b = 0;
  for (const auto& kv : m->ws.bufs) b += kv.second.cap;
  if (resident) *resident = b;
  if (allocs) *allocs = m->ws.allocs;
  API_END
}

int t0h_model_profile(t0h_model* m, int enable) {
  API_BEGIN
  require(m != nullptr, "t0h_model_profile: NULL model");
  bind_device(m);
  prof_collect(m);
  for (auto& e : m->prof.entries) {
    e.launches = 0;
    e.total_ms = 0.0;
  }
  m->prof.on = enable != 0;
  m->prof.only.clear();
  API_END
}

int t0h_model_profile_kind(t0h_model* m, const char* kind) {
  API_BEGIN
  require(m != nullptr && kind != nullptr, "t0h_model_profile_kind: NULL argument");
  require(kind[0] != '\0', "t0h_model_profile_kind: empty kind");
  bind_device(m);
  prof_collect(m);
  for (auto& e : m->prof.entries) {
    e.launches = 0;
    e.total_ms = 0.0;
  }
  m->prof.on = true;
  m->prof.only = kind;
  API_END
}

int t0h_model_profile_entry(t0h_model* m, size_t i, char* name, size_t name_cap, uint64_t* launches,
                            double* total_ms) {
  API_BEGIN
  require(m != nullptr, "t0h_model_profile_entry: NULL model");
  bind_device(m);
  prof_collect(m);
  if (i >= m->prof.entries.size()) throw Error(T0H_ERR_INVALID_ARG, "profile entry index out of range");
  const ProfEntry& e = m->prof.entries[i];
  if (name && name_cap) {
    std::snprintf(name, name_cap, "%s", e.name.c_str());
  }
  if (launches) *launches = e.launches;
  if (total_ms) *total_ms = e.total_ms;
  API_END
}

int t0h_model_graph_replay(t0h_model* m, int enable) {
  API_BEGIN
  require(m != nullptr, "t0h_model_graph_replay: NULL model");
  bind_device(m);
  if (!enable) {
    sync(m);
    destroy_graphs(m);
  }
  m->ws.graphs = enable != 0;
  API_END
}

int t0h_forward(t0h_model* m, const t0h_series* sr, float* out, size_t out_len, float* trace_pe, float* trace_l0) {
  API_BEGIN
  require(m && sr && out, "t0h_forward: NULL argument");
  require(sr->variates && sr->mask && sr->group_ids && sr->variate_type, "t0h_forward: NULL series array");
  bind_device(m);
  const t0h_config& c = m->mc.c;
  const int ps = (int)c.patch_size, nq = (int)c.n_quantiles, E = (int)c.embed_dim;
  if (sr->t % ps) throw Error(T0H_ERR_SHAPE, "series width must be patch-aligned");
  const int v = (int)sr->v, t = (int)sr->t, p = t / ps;
  check_out(out_len, (size_t)v * p * ps * nq);
  if (v == 0 || p == 0) return T0H_OK;
  check_window_rows(v, p);
  const size_t n = (size_t)v * t;
  for (size_t i = 0; i < n; ++i)
    if (sr->variate_type[i] >= m->n_types) throw Error(T0H_ERR_INVALID_ARG, "variate type out of range of the type embeddings");
  // dense group ids (negative stays padding) and the row-level grouping
  std::vector<int64_t> g(sr->group_ids, sr->group_ids + n), keys;
  for (int64_t x : g)
    if (x >= 0) keys.push_back(x);
  std::sort(keys.begin(), keys.end());
  keys.erase(std::unique(keys.begin(), keys.end()), keys.end());
  for (auto& x : g) x = x < 0 ? -1 : (int64_t)(std::lower_bound(keys.begin(), keys.end(), x) - keys.begin());
  std::vector<int64_t> row_group(v, -1);
  bool consistent = true;
  for (int r = 0; r < v && consistent; ++r)
    for (int i = 0; i < t; ++i) {
      const size_t k = (size_t)r * t + i;
      if (sr->mask[k] == T0H_MASK_PAD || g[k] < 0) continue;
      if (row_group[r] < 0) row_group[r] = g[k];
      else if (row_group[r] != g[k]) {
        consistent = false;
        break;
      }
    }
  const float* dv = put(m, "s_var", sr->variates, n);
  const int8_t* dm = put(m, "s_mask", sr->mask, n);
  const int64_t* dg = put(m, "s_grp", g.data(), n);
  const int64_t* dt = put(m, "s_type", sr->variate_type, n);
  upload_segments(m, row_group, consistent);
  PatchMeta pm = patch_buffers(m, v, p);
  SeriesDev sd{dv, dm, dg, dt, v, t, ps};
  PatchOut po{pm.enc_in, pm.grp, pm.att, pm.type_idx, pm.type_raw, pm.fut, nullptr, nullptr};
  launch_series_patchify(sd, po, m->stream);
  launch_fut_rows(pm.type_raw, pm.fut, v, p, m->stream);
  ensure_rope(m, p);
  encode_and_layers(m, v, p, pm, trace_pe, trace_l0);
  const int M = v * p;
  float* dout = decode_rows(m, M, RowGather{});
  float* q = ws_get<float>(m, "out", (size_t)M * ps * nq);
  launch_quantile_head(dout, q, M * ps, 1, nq, m->stream);
  download(m, out, q, (size_t)M * ps * nq);
  sync(m);
  (void)E;
  API_END
}

int t0h_forecast(t0h_model* m, const float* context, size_t v, size_t t_ctx, size_t horizon, float* out,
                 size_t out_len) {
  API_BEGIN
  require(m && context && out, "t0h_forecast: NULL argument");
  require(v > 0 && t_ctx > 0, "t0h_forecast: v and t_ctx must be positive");
  bind_device(m);
  check_out(out_len, v * horizon * m->mc.c.n_quantiles);
  forecast_host(m, context, v, t_ctx, horizon, out);
  API_END
}

int t0h_forecast_batch_chunked(t0h_model* m, const float* contexts, size_t n, size_t t_ctx, size_t horizon,
                               size_t chunk, float* out, size_t out_len) {
  API_BEGIN
  require(m && contexts && out, "t0h_forecast_batch_chunked: NULL argument");
  require(t_ctx > 0, "t0h_forecast_batch_chunked: t_ctx must be positive");
  bind_device(m);
  check_out(out_len, n * horizon * m->mc.c.n_quantiles);
  if (n == 0) return T0H_OK;
  forecast_batch_host(m, contexts, n, t_ctx, horizon, chunk, out);
  API_END
}

int t0h_forecast_batch_rows_chunked(t0h_model* m, const float* contexts, const size_t* lengths, size_t n,
                                    size_t horizon, size_t chunk, float* out, size_t out_len) {
  API_BEGIN
  require(m && out && (lengths || n == 0), "t0h_forecast_batch_rows_chunked: NULL argument");
  bind_device(m);
  const size_t nq = m->mc.c.n_quantiles, ps = m->mc.c.patch_size;
  check_out(out_len, n * horizon * nq);
  if (n == 0) return T0H_OK;
  size_t total = 0;
  std::vector<int64_t> offs(n);
  for (size_t i = 0; i < n; ++i) {
    offs[i] = (int64_t)total;
    total += lengths[i];
  }
  require(contexts || total == 0, "t0h_forecast_batch_rows_chunked: contexts is NULL");
  chunk = (chunk == 0 || chunk > n) ? n : chunk;
  numerics_begin(m);
  float* d_ctx = upload_contexts(m, contexts, total);
  float* d_out = ws_get<float>(m, "out", std::max<size_t>(1, n * horizon * nq));
  for (size_t start = 0; start < n; start += chunk) {  // lib.rs:200-240
    const size_t k = std::min(chunk, n - start);
    size_t common = 0;
    for (size_t r = 0; r < k; ++r) common = std::max(common, (lengths[start + r] + ps - 1) / ps * ps);
    WindowRows wr;
    wr.t_ctx = (int)common;
    wr.horizon = (int)horizon;
    wr.d_ctx = d_ctx;
    for (size_t r = 0; r < k; ++r) {
      wr.src_off.push_back(offs[start + r]);
      wr.len.push_back((int)lengths[start + r]);
      wr.group.push_back((int64_t)r);
    }
    forecast_window(m, wr, d_out + start * horizon * nq);
  }
  finish_host_call(m, out, d_out, n * horizon * nq);
  API_END
}

static void grouped_rows(WindowRows& wr, const int64_t* row_group, size_t n_rows, size_t t_ctx) {
  for (size_t r = 0; r < n_rows; ++r) {
    if (row_group[r] < 0) throw Error(T0H_ERR_INVALID_ARG, "group ids must be non-negative");
    wr.src_off.push_back((int64_t)(r * t_ctx));
    wr.len.push_back((int)t_ctx);
    wr.group.push_back(row_group[r]);
  }
}

int t0h_forecast_grouped(t0h_model* m, const float* contexts, const int64_t* row_group, size_t n_rows, size_t t_ctx,
                         size_t horizon, float* out, size_t out_len) {
  API_BEGIN
  require(m && contexts && row_group && out, "t0h_forecast_grouped: NULL argument");
  require(n_rows > 0 && t_ctx > 0, "t0h_forecast_grouped: n_rows and t_ctx must be positive");
  bind_device(m);
  const size_t nq = m->mc.c.n_quantiles;
  check_out(out_len, n_rows * horizon * nq);
  WindowRows wr;
  wr.t_ctx = (int)t_ctx;
  wr.horizon = (int)horizon;
  numerics_begin(m);
  wr.d_ctx = upload_contexts(m, contexts, n_rows * t_ctx);
  grouped_rows(wr, row_group, n_rows, t_ctx);
  float* d_out = ws_get<float>(m, "out", std::max<size_t>(1, n_rows * horizon * nq));
  forecast_window(m, wr, d_out);
  finish_host_call(m, out, d_out, n_rows * horizon * nq);
  API_END
}

int t0h_forecast_grouped_dev(t0h_model* m, const float* d_contexts, const int64_t* row_group, size_t n_rows,
                             size_t t_ctx, size_t horizon, float* d_out) {
  API_BEGIN
  require(m && d_contexts && row_group && d_out, "t0h_forecast_grouped_dev: NULL argument");
  require(n_rows > 0 && t_ctx > 0, "t0h_forecast_grouped_dev: n_rows and t_ctx must be positive");
  bind_device(m);
  WindowRows wr;
  wr.t_ctx = (int)t_ctx;
  wr.horizon = (int)horizon;
  wr.d_ctx = d_contexts;
  grouped_rows(wr, row_group, n_rows, t_ctx);
  m->nonfinite_unread = true;
  forecast_window(m, wr, d_out);
  API_END
}

int t0h_forecast_grouped_dev_noalloc(t0h_model* m, const float* d_contexts, const int64_t* row_group, size_t n_rows,
                                     size_t t_ctx, size_t horizon, float* d_out) {
  API_BEGIN
  require(m && d_contexts && row_group && d_out, "t0h_forecast_grouped_dev_noalloc: NULL argument");
  require(n_rows > 0 && t_ctx > 0, "t0h_forecast_grouped_dev_noalloc: n_rows and t_ctx must be positive");
  bind_device(m);
  WindowRows wr;
  wr.t_ctx = (int)t_ctx;
  wr.horizon = (int)horizon;
  wr.d_ctx = d_contexts;
  grouped_rows(wr, row_group, n_rows, t_ctx);
  // the previous call's copies out of the pinned staging must have executed
  if (m->noalloc_pending) {
    hip_check(hipEventSynchronize(m->noalloc_ev), "hipEventSynchronize");
    m->noalloc_pending = false;
  }
  Workspace::Arena& a = m->ws.arena;
  a.on = true;
  a.dev = static_cast<uint8_t*>(scratch_device_ptr(m->ctx->device));
  a.dev_cap = T0H_NOALLOC_SCRATCH_BYTES;
  a.dev_used = 0;
  a.host = static_cast<uint8_t*>(m->noalloc_host);
  a.host_cap = m->noalloc_host_bytes;
  a.host_used = 0;
  a.named.clear();
  struct Off {  // leave no-allocation mode on every exit
    t0h_model* m;
    ~Off() {
      Workspace::Arena& x = m->ws.arena;
      if (x.host_used && hipEventRecord(m->noalloc_ev, m->stream) == hipSuccess) m->noalloc_pending = true;
      x.on = false;
      x.named.clear();
    }
  } off{m};
  m->nonfinite_unread = true;
  forecast_window(m, wr, d_out);
  API_END
}

int t0h_model_check_numerics(t0h_model* m) {
  API_BEGIN
  require(m, "t0h_model_check_numerics: NULL model");
  bind_device(m);
  sync(m);
  m->nonfinite_unread = false;
  numerics_end(m);
  API_END
}

int t0h_forecast_grouped_ar(t0h_model* m, const float* contexts, const int64_t* row_group, size_t n_rows,
                            size_t t_ctx, size_t horizon, size_t steps, float* out, size_t out_len) {
  API_BEGIN
  require(m && contexts && row_group && out, "t0h_forecast_grouped_ar: NULL argument");
  require(n_rows > 0 && t_ctx > 0 && horizon > 0, "t0h_forecast_grouped_ar: sizes must be positive");
  bind_device(m);
  const size_t nq = m->mc.c.n_quantiles;
  check_out(out_len, n_rows * steps * horizon * nq);
  if (steps == 0) return T0H_OK;
  const int qi = median_index(m->mc.c);
  numerics_begin(m);
  float* ctx_a = put(m, "ar_ctx_a", contexts, n_rows * t_ctx);
  float* ctx_b = ws_get<float>(m, "ar_ctx_b", n_rows * t_ctx);
  float* step_out = ws_get<float>(m, "ar_step", n_rows * horizon * nq);
  float* result = ws_get<float>(m, "ar_out", n_rows * steps * horizon * nq);
  for (size_t st = 0; st < steps; ++st) {
    WindowRows wr;
    wr.t_ctx = (int)t_ctx;
    wr.horizon = (int)horizon;
    wr.d_ctx = ctx_a;
    grouped_rows(wr, row_group, n_rows, t_ctx);
    forecast_window(m, wr, step_out);
    launch_ar_store(result, step_out, (int)n_rows, (int)horizon, (int)nq, (int)steps, (int)st, m->stream);
    launch_ar_shift(ctx_b, ctx_a, step_out, (int)n_rows, (int)t_ctx, (int)horizon, (int)nq, qi, m->stream);
    std::swap(ctx_a, ctx_b);
  }
  finish_host_call(m, out, result, n_rows * steps * horizon * nq);
  API_END
}

int t0h_forecast_rollout(t0h_model* m, const float* context, size_t t_ctx, size_t prediction_length,
                         const float* query, size_t n_query, float* out, size_t out_len) {
  API_BEGIN
  require(m && context && query && out, "t0h_forecast_rollout: NULL argument");
  require(t_ctx > 0 && n_query > 0, "t0h_forecast_rollout: t_ctx and n_query must be positive");
  bind_device(m);
  check_out(out_len, prediction_length * n_query);
  // model.rs:582-665 / lib.rs:259-341
  const t0h_config& c = m->mc.c;
  const size_t ps = c.patch_size, nt = c.n_quantiles;
  const std::vector<float> q(query, query + n_query);
  const std::vector<float> trained_mass = prob_mass(c.quantile_levels, nt);
  const std::vector<float> query_mass = prob_mass(query, n_query);
  const size_t context_width = (t_ctx + ps - 1) / ps * ps;
  const size_t horizon0 = std::min<size_t>((prediction_length + ps - 1) / ps * ps, T0H_MAX_HORIZON);
  std::vector<float> block0(horizon0 * nt);
  forecast_host(m, context, 1, t_ctx, horizon0, block0.data());
  std::vector<float> first;
  for (size_t h = 0; h < horizon0; ++h) {
    auto r = interpolate_quantiles(q, c.quantile_levels, block0.data() + h * nt, nt);
    first.insert(first.end(), r.begin(), r.end());
  }
  std::vector<float> all(first);
  if (prediction_length > horizon0) {
    const size_t n_paths = n_query;
    std::vector<std::vector<float>> paths(n_paths, std::vector<float>(context, context + t_ctx));
    size_t remaining = prediction_length - horizon0;
    std::vector<float> prev = first;
    size_t prev_width = horizon0;
    std::vector<float> weights(n_paths * nt), samples(n_paths * nt);
    for (size_t j = 0; j < n_paths; ++j)
      for (size_t pq = 0; pq < nt; ++pq) weights[j * nt + pq] = trained_mass[pq] * query_mass[j];
    while (remaining > 0) {
      for (size_t j = 0; j < n_paths; ++j)
        for (size_t h = 0; h < prev_width; ++h) paths[j].push_back(prev[h * n_query + j]);
      const size_t horizon = std::min<size_t>((remaining + ps - 1) / ps * ps, T0H_MAX_HORIZON);
      std::vector<float> bctx(n_paths * context_width, 0.0f);
      for (size_t j = 0; j < n_paths; ++j) {
        const size_t wl = std::min(context_width, paths[j].size());
        std::copy(paths[j].end() - wl, paths[j].end(), bctx.begin() + j * context_width + (context_width - wl));
        // keep only what a future window can reach
        if (paths[j].size() > 4 * context_width) paths[j].erase(paths[j].begin(), paths[j].end() - context_width);
      }
      std::vector<float> blocks(n_paths * horizon * nt);
      forecast_batch_host(m, bctx.data(), n_paths, context_width, horizon, n_paths, blocks.data());
      std::vector<float> reduced;
      for (size_t h = 0; h < horizon; ++h) {
        for (size_t j = 0; j < n_paths; ++j)
          for (size_t pq = 0; pq < nt; ++pq) samples[j * nt + pq] = blocks[j * horizon * nt + h * nt + pq];
        auto r = weighted_quantile(q, weights, samples);
        reduced.insert(reduced.end(), r.begin(), r.end());
      }
      all.insert(all.end(), reduced.begin(), reduced.end());
      prev = reduced;
      prev_width = horizon;
      remaining = remaining > horizon ? remaining - horizon : 0;  // saturating_sub (model.rs:660)
    }
  }
  std::copy(all.begin(), all.begin() + prediction_length * n_query, out);
  API_END
}

int t0h_dequant(int qtype, const void* d_blocks, size_t n, float* d_out, void* stream) {
  API_BEGIN
  launch_dequant(qtype, d_blocks, n, d_out, static_cast<hipStream_t>(stream));
  API_END
}

// The kernel-level entry points' operands: the kernels move weights, activations and outputs in
// 16-byte vectors, so the base pointers must be 16-byte aligned (as hipMalloc returns them).
static bool gemm_ptrs_aligned(const void* w, const void* x, const void* y, const void* bias) {
  auto a = [](const void* p, uintptr_t m) { return (reinterpret_cast<uintptr_t>(p) & (m - 1)) == 0; };
  return a(w, 16) && a(x, 16) && a(y, 16) && a(bias, 4);
}

int t0h_gemm_q(int wtype, const void* d_w, const float* d_x, const float* d_bias, float* d_y, size_t m, size_t n,
               size_t k, int act, void* stream) {
  API_BEGIN
  require(m < (1u << 31) && n < (1u << 31) && k < (1u << 31), "t0h_gemm_q: dimension too large");
  require(gemm_ptrs_aligned(d_w, d_x, d_y, d_bias), "t0h_gemm_q: d_w, d_x and d_y must be 16-byte aligned");
  GemmDesc d;
  d.wtype = wtype;
  d.w = d_w;
  d.a = d_x;
  d.a_f32 = 1;
  d.lda = (int)k;
  d.bias = d_bias;
  d.y = d_y;
  d.ldy = (int)n;
  d.M = (int)m;
  d.N = (int)n;
  d.K = (int)k;
  d.relu = act == 1;
  d.epi = EPI_STORE_F32;
  launch_gemm(d, static_cast<hipStream_t>(stream));
  API_END
}

int t0h_gemm_f16(int wtype, const void* d_w, const void* d_x, const float* d_bias, void* d_y, size_t m, size_t n,
                 size_t k, int epilogue, int tile, void* stream) {
  API_BEGIN
  require(m < (1u << 31) && n < (1u << 31) && k < (1u << 31), "t0h_gemm_f16: dimension too large");
  require(epilogue >= EPI_STORE_F32 && epilogue <= EPI_SWIGLU_F16, "t0h_gemm_f16: unknown epilogue");
  require(tile >= 0 && tile <= 8 && tile != 2, "t0h_gemm_f16: tile must be 0, 1 or 3..8");
  require(gemm_ptrs_aligned(d_w, d_x, d_y, d_bias), "t0h_gemm_f16: d_w, d_x and d_y must be 16-byte aligned");
  GemmDesc d;
  d.wtype = wtype;
  d.w = d_w;
  d.a = d_x;
  d.a_f32 = 0;
  d.lda = (int)k;
  d.bias = d_bias;
  d.y = d_y;
  d.ldy = (int)n;
  d.M = (int)m;
  d.N = (int)n;
  d.K = (int)k;
  d.epi = epilogue;
  launch_gemm_forced(d, tile == 0 ? 0 : tile + 2, static_cast<hipStream_t>(stream));
  API_END
}

size_t t0h_row_bytes(int qtype, size_t n) { return row_bytes(qtype, n); }

int t0h_quantize(int qtype, const float* x, size_t n, uint8_t* out, size_t out_len) {
  API_BEGIN
  const size_t nb = row_bytes(qtype, n);
  if (nb == 0 && n != 0) throw Error(T0H_ERR_SHAPE, "quantize: element count is not a multiple of 32");
  require(out_len >= nb, "quantize: output buffer too small");
  require((x && out) || n == 0, "quantize: NULL argument");
  quantize(qtype, x, n, out);
  API_END
}

int t0h_synth_model_gguf(const t0h_synth_spec* spec, int quant, uint8_t* out, size_t cap, size_t* len) {
  API_BEGIN
  require(spec && len, "t0h_synth_model_gguf: NULL argument");
  std::vector<uint8_t> b = synth_model_gguf(*spec, quant);
  *len = b.size();
  if (out) {
    require(cap >= b.size(), "t0h_synth_model_gguf: output buffer too small");
    std::memcpy(out, b.data(), b.size());
  }
  API_END
}

int t0h_export_gguf_from_safetensors(const uint8_t* st, size_t st_len, const char* config_json, int quant,
                                     uint8_t* out, size_t cap, size_t* out_len) {
  API_BEGIN
  require(st && config_json && out_len, "t0h_export_gguf_from_safetensors: NULL argument");
  std::vector<uint8_t> b = export_gguf_from_safetensors(st, st_len, config_json, quant);
  *out_len = b.size();
  if (out) {
    require(cap >= b.size(), "t0h_export_gguf_from_safetensors: output buffer too small");
    std::memcpy(out, b.data(), b.size());
  }
  API_END
}

int t0h_model_load_safetensors(t0h_ctx* ctx, const uint8_t* st, size_t st_len, const char* config_json, int quant,
                               t0h_model** out) {
  API_BEGIN
  require(ctx && st && config_json && out, "t0h_model_load_safetensors: NULL argument");
  *out = nullptr;
  const std::vector<uint8_t> g = export_gguf_from_safetensors(st, st_len, config_json, quant);
  const int rc = t0h_model_load_gguf(ctx, g.data(), g.size(), out);
  if (rc) return rc;  // the message is already set
  API_END
}

int t0h_export_gguf(const uint8_t* bytes, size_t len, int quant, uint8_t* out, size_t cap, size_t* out_len) {
  API_BEGIN
  require(bytes && out_len, "t0h_export_gguf: NULL argument");
  std::vector<uint8_t> b = export_gguf(bytes, len, quant);
  *out_len = b.size();
  if (out) {
    require(cap >= b.size(), "t0h_export_gguf: output buffer too small");
    std::memcpy(out, b.data(), b.size());
  }
  API_END
}

}  // extern "C"
