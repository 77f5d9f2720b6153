// mmf_host.cpp -- host side of libmmfree_hip.so: the C ABI of include/mmfree_hip.h.
//
// Owns the device state of one engine instance: resident 2-bit projections, the model's
// fp32 tensors, the recurrent state and scratch, and the single-row decode plan (4 fused
// launches per layer + the lm_head, captured once into a HIP graph and replayed per
// token). Prefill, batched serving steps and the stateless forward run the row kernels.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/mmfree_hip.h"
#include "mmf_internal.hpp"

using namespace mmf;

namespace {

struct Err {
  int code;
  std::string msg;
};

#define MMF_HIP(expr)                                                                     \
  do {                                                                                    \
    hipError_t e_ = (expr);                                                               \
    if (e_ != hipSuccess)                                                                 \
      throw Err{MMF_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(e_)};          \
  } while (0)

[[noreturn]] void fail(int code, const std::string& m) { throw Err{code, m}; }

// Grow-only device buffer. Every reallocation bumps dbuf_epoch, so a captured graph that
// baked in buffer addresses can tell that it is stale.
std::atomic<uint64_t> dbuf_epoch{0};

struct DBuf {
  void* p = nullptr;
  size_t n = 0;
  void* get(size_t bytes) {
    if (bytes > n) {
      if (p) MMF_HIP(hipFree(p));
      p = nullptr;
      n = 0;
      MMF_HIP(hipMalloc(&p, bytes));
      n = bytes;
      ++dbuf_epoch;
    }
    return p;
  }
  template <class T> T* as(size_t count) { return static_cast<T*>(get(count * sizeof(T))); }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    n = 0;
  }
};

// Grow-only pinned host buffer (hipHostMalloc) for copies that must not stage through
// pageable memory.
struct PinBuf {
  void* p = nullptr;
  size_t n = 0;
  void* get(size_t bytes) {
    if (bytes > n) {
      if (p) (void)hipHostFree(p);
      p = nullptr;
      n = 0;
      MMF_HIP(hipHostMalloc(&p, bytes, hipHostMallocDefault));
      n = bytes;
    }
    return p;
  }
  template <class T> T* as(size_t count) { return static_cast<T*>(get(count * sizeof(T))); }
  void release() {
    if (p) (void)hipHostFree(p);
    p = nullptr;
    n = 0;
  }
};

struct Proj {
  ProjDev d;
  void* mem = nullptr;   // pk | tail | rowsum | normw in one allocation
  void* mem4 = nullptr;  // pk4 (float-mode models only)
};

struct DevTensor {
  void* p = nullptr;
  std::vector<size_t> shape;
  int dtype = 0;  // 0 f32, 1 i8
  int proj = -1;  // for ".wq": index into ctx->projs
  std::vector<float> host_small;  // f32 tensors of <= 16 elements (scale_w)
  size_t numel() const {
    size_t n = 1;
    for (auto s : shape) n *= s;
    return shape.empty() ? 0 : n;
  }
};

struct LayerDev {
  int proj[6];
  const float *attn = nullptr, *mlp = nullptr, *gn = nullptr, *lb = nullptr;
  const float *attnT = nullptr, *mlpT = nullptr, *gnT = nullptr;  // chain-transposed
};

// Scratch for row (multi-token) passes.
struct RowScratch {
  DBuf ids, h, resid, i, f, g, recur, scan, z, logits, state0, am;
  DBuf acty, actq, actct, actsa;
  DBuf segs;  // stacked prompts: nseg + 1 row offsets, then the nseg last-row indices
  DBuf chunk;  // chunk summaries and starting states of the chunked scan
};

struct Model {
  mmf_config cfg{};
  bool begun = false, finalized = false;
  int mode = kFloat, frac = 10;
  float qs = 1024.0f;
  bool chunked_scan = false;  // float prefill: chunked parallel scan (mmf_model_set_scan)
  std::unordered_map<std::string, DevTensor> tensors;
  const float* emb = nullptr;
  const float* norm_w = nullptr;
  const float* norm_wT = nullptr;
  int lm = -1;
  std::vector<LayerDev> layers;
  Geom gH{}, gI{};  // chain geometry of H- and I-long vectors
  DBuf embT, normT;  // chain-transposed embedding table and norm weights
  // decode buffers (single row, chain-transposed)
  DBuf h, resid, g, recur, z, logits, key, hist, hist_pos;
  size_t hist_cap = 0;
  DBuf state;  // [L][B][H]
  size_t streams = 0;
  RowScratch rs;
  // decode graph
  hipGraphExec_t graph = nullptr;
  bool graph_tried = false;
  // batched serving step graph, valid for step_B streams while no buffer moved
  hipGraphExec_t step_graph = nullptr;
  size_t step_B = 0;
  uint64_t step_epoch = 0;
  // external integer matmul of the FixedQ510 projections (mmf_model_set_matmul)
  mmf_matmul_fn ext_fn = nullptr;
  void* ext_user = nullptr;
  DBuf ext_codes, ext_acc;
  std::vector<int32_t> ext_hcodes, ext_hacc;
  bool ext_on() const { return ext_fn && mode == kFixed; }
};

// Optional per-launch timing of the row path: an event pair around each launch, summed
// per kind after the run (the elapsed time of a pair is that kernel's execution on the
// stream, independent of host submission gaps).
enum RowKind : int { kRkPrologue, kRkGemmIFG, kRkMixer, kRkGemmO, kRkGemmGate, kRkGemmDown, kRkLM, kRkOther,
                     kRkCount };

struct RowTimer {
  bool on = false;
  std::vector<hipEvent_t> pool;
  std::vector<int> kinds;  // kind of event pair i (events 2i, 2i+1)
  size_t used = 0;
  hipEvent_t take() {
    if (used == pool.size()) {
      hipEvent_t e;
      MMF_HIP(hipEventCreate(&e));
      pool.push_back(e);
    }
    return pool[used++];
  }
  ~RowTimer() {
    for (auto e : pool) (void)hipEventDestroy(e);
  }
};

}  // namespace

struct mmf_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string err;
  std::vector<Proj> projs;
  Model model;
  DBuf raw;  // staging for int8 weights before the repack
  DBuf opy, opq, opct, opsa, opstate;
  DBuf gws;  // split-K workspace of the matrix-core GEMM
  DBuf hmx, hmacc;        // mmf_ternary_matmul_host: codes and accumulators on the device
  PinBuf pin_x, pin_acc;  // ... and their pinned host staging
  hipDeviceProp_t prop{};
  RowTimer timer;
};

namespace {

thread_local std::string g_create_err;

template <class F>
int guard(mmf_ctx* ctx, F&& f) {
  if (!ctx) return MMF_ERR_ARG;
  try {
    MMF_HIP(hipSetDevice(ctx->device));
    f();
    return MMF_OK;
  } catch (const Err& e) {
    ctx->err = e.msg;
    return e.code;
  } catch (const std::bad_alloc&) {
    ctx->err = "out of host memory";
    return MMF_ERR_ARG;
  } catch (const std::exception& e) {
    ctx->err = e.what();
    return MMF_ERR_ARG;
  }
}

const Proj& proj_of(mmf_ctx* c, int id) {
  if (id < 0 || id >= static_cast<int>(c->projs.size())) fail(MMF_ERR_ARG, "invalid proj_id " + std::to_string(id));
  if (!c->projs[id].mem) fail(MMF_ERR_ARG, "proj_id " + std::to_string(id) + " was released");
  return c->projs[id];
}

float inv_fixed_of(float scale_w, int frac) {
  const float qs = static_cast<float>(1u << frac);
  return 1.0f / (qs * scale_w);  // bitlinear.cpp:29-30
}

int register_proj(mmf_ctx* c, const int8_t* wq_dev, size_t N, size_t K, float scale_w, const float* normw_host,
                  const float* normw_dev) {
  if (N == 0 || K == 0 || N > (1u << 30) || K > (1u << 20)) fail(MMF_ERR_ARG, "invalid projection shape");
  Proj P;
  P.d.g = make_geom(static_cast<int>(N), static_cast<int>(K));
  const Geom& g = P.d.g;
  const size_t words = static_cast<size_t>(g.ngroups) * g.Wc * kGroup * 8;
  const size_t npad = static_cast<size_t>(g.ngroups) * kGroup;
  const size_t b_pk = words * 4, b_tail = npad * 8, b_rs = npad * 4, b_nw = normw_host ? K * 4 : 0;
  const size_t b_nwT = normw_host ? (8 * static_cast<size_t>(g.Lc) + 8) * 4 : 0;  // chain-transposed copy
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  const size_t b_pkm = pkm_words(g) * 4;
  MMF_HIP(hipMalloc(&P.mem, al(b_pk) + al(b_pkm) + al(b_tail) + al(b_rs) + al(b_nw) + al(b_nwT) + 256));
  char* base = static_cast<char*>(P.mem);
  P.d.pk = reinterpret_cast<uint32_t*>(base);
  P.d.pkm = reinterpret_cast<uint32_t*>(base + al(b_pk));
  base += al(b_pkm);
  P.d.tail = reinterpret_cast<int8_t*>(base + al(b_pk));
  P.d.rowsum = reinterpret_cast<int32_t*>(base + al(b_pk) + al(b_tail));
  float* nw = reinterpret_cast<float*>(base + al(b_pk) + al(b_tail) + al(b_rs));
  if (normw_host) {
    MMF_HIP(hipMemcpy(nw, normw_host, b_nw, hipMemcpyHostToDevice));
    P.d.normw = nw;
    float* nwT = reinterpret_cast<float*>(reinterpret_cast<char*>(nw) + al(b_nw));
    MMF_HIP(launch_to_chain(nw, nwT, 1, static_cast<int>(K), g.Lc, c->stream));
    P.d.normwT = nwT;
  } else {
    P.d.normw = normw_dev;
  }
  P.d.scale_w = scale_w;
  P.d.inv_scale_w = 1.0f / scale_w;  // bitlinear.cpp:28
  P.d.inv_fixed = inv_fixed_of(scale_w, 10);
  hipError_t e = launch_pack(wq_dev, g, const_cast<uint32_t*>(P.d.pk), const_cast<int8_t*>(P.d.tail),
                             const_cast<int32_t*>(P.d.rowsum), c->stream);
  if (e == hipErrorInvalidValue) {
    (void)hipFree(P.mem);
    fail(MMF_ERR_ARG, "projection weights must be ternary (-1, 0, +1)");
  }
  MMF_HIP(e);
  MMF_HIP(launch_pack_mfma(P.d.pk, g, false, const_cast<uint32_t*>(P.d.pkm), c->stream));
  c->projs.push_back(P);
  return static_cast<int>(c->projs.size() - 1);
}

// The fp4 slab of a projection for the float-mode decode kernels, built once from its 2-bit slab.
void ensure_pk4(mmf_ctx* c, Proj& P) {
  if (P.d.pk4) return;
  MMF_HIP(hipMalloc(&P.mem4, pk4_words(P.d.g) * 4));
  MMF_HIP(launch_pack4(P.d.pk, P.d.g, static_cast<uint32_t*>(P.mem4), c->stream));
  P.d.pk4 = static_cast<const uint32_t*>(P.mem4);
}

void tbeg(mmf_ctx* c, int kind) {
  if (!c->timer.on) return;
  c->timer.kinds.push_back(kind);
  MMF_HIP(hipEventRecord(c->timer.take(), c->stream));
}
void tend(mmf_ctx* c) {
  if (c->timer.on) MMF_HIP(hipEventRecord(c->timer.take(), c->stream));
}

// ---- activation buffers ---------------------------------------------------------------
// Geometry of the activations of `rows` rows for na projections, no buffers attached.
ActBuf act_shape(const Geom& g, int rows, int na) {
  ActBuf a;
  a.Lc = g.Lc;
  a.K = g.K;
  a.K8 = g.K8;
  a.nb = g.nb;
  a.ntail = g.ntail;
  a.rows = rows;
  a.na = na;
  return a;
}

// Bytes of the buffers y, q, ct, sa that `mode` uses for the activations a (0 if unused).
void act_bytes(Mode mode, const ActBuf& a, size_t out[4]) {
  const size_t nr = static_cast<size_t>(a.rows) * a.na;
  out[0] = mode == kFloat ? nr * a.ystride() * sizeof(float) : 0;
  out[1] = mode == kFloat ? 0 : 2 * static_cast<size_t>(a.na) * a.qplane();
  out[2] = mode == kFloat ? 0 : nr * 8 * sizeof(int32_t);
  out[3] = mode == kFloat ? 0 : nr * sizeof(float);
}

ActBuf make_act(DBuf& y, DBuf& q, DBuf& ct, DBuf& sa, Mode mode, const Geom& g, int rows, int na) {
  ActBuf a = act_shape(g, rows, na);
  size_t b[4];
  act_bytes(mode, a, b);
  if (mode == kFloat) {
    a.y = static_cast<float*>(y.get(b[0]));
  } else {
    a.q = static_cast<int8_t*>(q.get(b[1]));
    a.ct = static_cast<int32_t*>(ct.get(b[2]));
    a.sa = static_cast<float*>(sa.get(b[3]));
  }
  return a;
}

// launch_gemm with the split-K workspace it asks for (grow-only, owned by the context).
void run_gemm(mmf_ctx* c, GemmArgs& ga, const ActBuf& act, hipStream_t st) {
  const size_t wsb = gemm_workspace_bytes(ga);
  ga.ws = wsb ? static_cast<int32_t*>(c->gws.get(wsb)) : nullptr;
  MMF_HIP(launch_gemm(ga, act, st));
}

GemmArgs gemm_args(mmf_ctx* c, const int* ids, int n, int rows, Mode mode, int frac) {
  GemmArgs a{};
  a.nmat = n;
  a.rows = rows;
  a.mode = mode;
  for (int z = 0; z < n; ++z) {
    a.p[z] = proj_of(c, ids[z]).d;
    a.inv_fixed[z] = inv_fixed_of(a.p[z].scale_w, frac);
  }
  a.epi = kEpiStore;
  return a;
}

// One projection group of the model: the built-in GEMM, or, with an external integer matmul
// set in FixedQ510, codes to the host, the caller's accumulators back, and the same
// dequantisation and output stage on the device (layer/proj as mmf_model_set_matmul names
// them).
void proj_gemm(mmf_ctx* c, Model& m, GemmArgs& ga, const ActBuf& act, hipStream_t st, int layer, int proj) {
  if (!m.ext_on()) {
    run_gemm(c, ga, act, st);
    return;
  }
  const size_t k = ga.nmat, rows = ga.rows, K = act.K, N = ga.p[0].g.N;
  int32_t* dcodes = m.ext_codes.as<int32_t>(k * rows * K);
  int32_t* dacc = m.ext_acc.as<int32_t>(k * rows * N);
  m.ext_hcodes.resize(k * rows * K);
  m.ext_hacc.assign(k * rows * N, 0);
  MMF_HIP(launch_planes_to_codes(act, kFixed, dcodes, st));
  MMF_HIP(hipMemcpyAsync(m.ext_hcodes.data(), dcodes, k * rows * K * sizeof(int32_t), hipMemcpyDeviceToHost, st));
  MMF_HIP(hipStreamSynchronize(st));
  const int rc = m.ext_fn(m.ext_user, layer, proj, static_cast<int>(k), m.ext_hcodes.data(), m.ext_hacc.data(), K, N,
                          rows);
  if (rc != 0)
    fail(MMF_ERR_ARG, "external matmul of layer " + std::to_string(layer) + " projection " + std::to_string(proj) +
                          " failed (" + std::to_string(rc) + ")");
  MMF_HIP(hipMemcpyAsync(dacc, m.ext_hacc.data(), k * rows * N * sizeof(int32_t), hipMemcpyHostToDevice, st));
  ga.ws = dacc;
  MMF_HIP(launch_acc_epilogue(ga, act, st));
  // the host arrays are reused by the next projection: wait for the upload
  MMF_HIP(hipStreamSynchronize(st));
}

// ---- model helpers -------------------------------------------------------------------
Model& model_of(mmf_ctx* c) {
  if (!c->model.finalized) fail(MMF_ERR_STATE, "no model: call mmf_model_begin/tensor/finalize first");
  return c->model;
}

const DevTensor& tensor_of(Model& m, const std::string& name) {
  auto it = m.tensors.find(name);
  if (it == m.tensors.end()) fail(MMF_ERR_MISSING, "weights: missing tensor " + name);
  return it->second;
}

void check_shape(const DevTensor& t, const std::string& name, std::vector<size_t> want) {
  if (t.shape != want) {
    std::string s = "weights: tensor " + name + " has shape [";
    for (size_t i = 0; i < t.shape.size(); ++i) s += (i ? "," : "") + std::to_string(t.shape[i]);
    fail(MMF_ERR_ARG, s + "], expected another");
  }
}

void check_ids(const Model& m, const int64_t* ids, size_t n) {
  for (size_t i = 0; i < n; ++i)
    if (ids[i] < 0 || static_cast<size_t>(ids[i]) >= m.cfg.vocab_size)
      fail(MMF_ERR_ARG, "token id " + std::to_string(ids[i]) + " outside the vocabulary");
}

size_t chain_len(const Geom& g) { return static_cast<size_t>(8 * g.Lc + 8); }

void alloc_decode(mmf_ctx* c, Model& m) {
  const size_t WH = chain_len(m.gH), WI = chain_len(m.gI), V = m.cfg.vocab_size;
  for (DBuf* b : {&m.h, &m.resid, &m.g, &m.recur}) {
    b->as<float>(WH);
    MMF_HIP(hipMemsetAsync(b->p, 0, WH * sizeof(float), c->stream));  // zero padding
  }
  m.z.as<float>(WI);
  MMF_HIP(hipMemsetAsync(m.z.p, 0, WI * sizeof(float), c->stream));
  m.logits.as<float>(V);
  m.key.as<unsigned long long>(kLMBlocks);
  m.hist_pos.as<int32_t>(1);
}

// One layer over `rows` rows with the row kernels. h [rows, H] in/out; state: this
// layer's state ([H] time scan or [rows, H] streams); internals (may be null): device
// [5][rows][H] copy targets for the trace.
void layer_rows(mmf_ctx* c, Model& m, int l, int rows, float* h, float* state, bool stream_state,
                float* trace_dev, const int* segs = nullptr, int nseg = 0) {
  const int H = static_cast<int>(m.cfg.hidden_size), I = static_cast<int>(m.cfg.intermediate_size);
  const Mode mode = static_cast<Mode>(m.mode);
  const LayerDev& L = m.layers[l];
  RowScratch& s = m.rs;
  hipStream_t st = c->stream;
  float* ib = s.i.as<float>(static_cast<size_t>(rows) * H);
  float* fb = s.f.as<float>(static_cast<size_t>(rows) * H);
  float* gb = s.g.as<float>(static_cast<size_t>(rows) * H);
  float* rb = s.recur.as<float>(static_cast<size_t>(rows) * H);
  float* resid = s.resid.as<float>(static_cast<size_t>(rows) * H);
  float* zb = s.z.as<float>(static_cast<size_t>(rows) * I * 2);
  float* scan = (trace_dev || segs || (!stream_state && rows > 1)) ? s.scan.as<float>(static_cast<size_t>(rows) * H)
                                                                   : nullptr;

  // attention: attn_norm -> i/f/g BitLinears (hgrn_model.cpp:95-107)
  {
    const Geom& g = proj_of(c, L.proj[0]).d.g;
    ActBuf act = make_act(s.acty, s.actq, s.actct, s.actsa, mode, g, rows, 3);
    PrologueArgs pa{};
    pa.x = h;
    pa.pre = kPreNorm;
    pa.pre_w = L.attn;
    pa.pre_wT = L.attnT;
    pa.na = 3;
    for (int k = 0; k < 3; ++k) {
      pa.normw[k] = proj_of(c, L.proj[k]).d.normw;
      pa.normwT[k] = proj_of(c, L.proj[k]).d.normwT;
    }
    pa.eps = m.cfg.rms_norm_eps;
    pa.qs = m.qs;
    tbeg(c, kRkPrologue);
    MMF_HIP(launch_prologue(mode, pa, act, st));
    tend(c);
    GemmArgs ga = gemm_args(c, L.proj, 3, rows, mode, m.frac);
    ga.out[0] = ib;
    ga.out[1] = fb;
    ga.out[2] = gb;
    tbeg(c, kRkGemmIFG);
    proj_gemm(c, m, ga, act, st, l, 0);
    tend(c);
  }
  // gate, lower bound, swiglu, recurrence (hgrn_model.cpp:109-150). Independent streams
  // without a trace: the step runs inside the g_norm prologue below (kPreMixSwish), which
  // reports hipErrorNotSupported, launching nothing, where its float4 form does not apply.
  const bool mix_in_prologue = stream_state && !segs && !trace_dev;
  auto run_mixer = [&]() -> hipError_t {
    tbeg(c, kRkMixer);
    const hipError_t e = segs ? launch_mixer_segs(ib, fb, scan, rb, state, L.lb, segs, nseg, rows, H,
                                                  trace_dev != nullptr, st)
                              : launch_mixer(ib, fb, scan, rb, state, L.lb, rows, H, stream_state,
                                             trace_dev != nullptr, st);
    tend(c);
    return e;
  };
  // float mode, opt-in: the chunked parallel scan instead of the time-ordered one (a prefill
  // of one sequence without a trace; H % 64 == 0)
  const bool chunked = mode == kFloat && m.chunked_scan && !stream_state && !segs && !trace_dev && rows > 1 &&
                       H % 64 == 0;
  if (chunked) {
    tbeg(c, kRkMixer);
    float* ws = s.chunk.as<float>(scan_chunked_ws_floats(rows, H));
    MMF_HIP(launch_scan_chunked(ib, fb, L.lb, rb, state, ws, rows, H, st));
    tend(c);
  } else if (!mix_in_prologue) {
    MMF_HIP(run_mixer());
  }
  if (trace_dev) {
    const size_t n = static_cast<size_t>(rows) * H * sizeof(float);
    MMF_HIP(hipMemcpyAsync(trace_dev + 0 * rows * H, ib, n, hipMemcpyDeviceToDevice, st));
    MMF_HIP(hipMemcpyAsync(trace_dev + 1 * rows * H, fb, n, hipMemcpyDeviceToDevice, st));
    MMF_HIP(hipMemcpyAsync(trace_dev + 2 * rows * H, gb, n, hipMemcpyDeviceToDevice, st));
    MMF_HIP(hipMemcpyAsync(trace_dev + 3 * static_cast<size_t>(rows) * H, scan, n, hipMemcpyDeviceToDevice, st));
    MMF_HIP(hipMemcpyAsync(trace_dev + 4 * static_cast<size_t>(rows) * H, rb, n, hipMemcpyDeviceToDevice, st));
  }
  // g_norm -> o_proj -> resid = h + o (hgrn_model.cpp:153-166)
  {
    const Geom& g = proj_of(c, L.proj[3]).d.g;
    ActBuf act = make_act(s.acty, s.actq, s.actct, s.actsa, mode, g, rows, 1);
    PrologueArgs pa{};
    pa.x = gb;
    pa.x2 = rb;
    pa.pre = kPreSwish;
    pa.pre_w = L.gn;
    pa.pre_wT = L.gnT;
    pa.na = 1;
    pa.normw[0] = proj_of(c, L.proj[3]).d.normw;
    pa.normwT[0] = proj_of(c, L.proj[3]).d.normwT;
    pa.eps = m.cfg.rms_norm_eps;
    pa.qs = m.qs;
    bool done = false;
    if (mix_in_prologue) {
      PrologueArgs pm = pa;
      pm.pre = kPreMixSwish;
      pm.x2 = ib;
      pm.mix_f = fb;
      pm.mix_state = state;
      pm.mix_lb = L.lb;
      tbeg(c, kRkPrologue);
      const hipError_t e = launch_prologue(mode, pm, act, st);
      tend(c);
      if (e != hipErrorNotSupported) {
        MMF_HIP(e);
        done = true;
      } else {
        MMF_HIP(run_mixer());
      }
    }
    if (!done) {
      tbeg(c, kRkPrologue);
      MMF_HIP(launch_prologue(mode, pa, act, st));
      tend(c);
    }
    GemmArgs ga = gemm_args(c, &L.proj[3], 1, rows, mode, m.frac);
    ga.epi = kEpiAdd;
    ga.add = h;
    ga.out[0] = resid;
    tbeg(c, kRkGemmO);
    proj_gemm(c, m, ga, act, st, l, 3);
    tend(c);
  }
  // mlp_norm -> gate_proj -> swiglu (hgrn_model.cpp:167-185)
  {
    const Geom& g = proj_of(c, L.proj[4]).d.g;
    ActBuf act = make_act(s.acty, s.actq, s.actct, s.actsa, mode, g, rows, 1);
    PrologueArgs pa{};
    pa.x = resid;
    pa.pre = kPreNorm;
    pa.pre_w = L.mlp;
    pa.pre_wT = L.mlpT;
    pa.na = 1;
    pa.normw[0] = proj_of(c, L.proj[4]).d.normw;
    pa.normwT[0] = proj_of(c, L.proj[4]).d.normwT;
    pa.eps = m.cfg.rms_norm_eps;
    pa.qs = m.qs;
    tbeg(c, kRkPrologue);
    MMF_HIP(launch_prologue(mode, pa, act, st));
    tend(c);
    GemmArgs ga = gemm_args(c, &L.proj[4], 1, rows, mode, m.frac);
    ga.epi = kEpiSwigluPair;
    ga.out[0] = zb;
    ga.swiglu_n = rows * I;
    tbeg(c, kRkGemmGate);
    proj_gemm(c, m, ga, act, st, l, 4);
    tend(c);
  }
  // down_proj -> h = resid + d (hgrn_model.cpp:187-194)
  {
    const Geom& g = proj_of(c, L.proj[5]).d.g;
    ActBuf act = make_act(s.acty, s.actq, s.actct, s.actsa, mode, g, rows, 1);
    PrologueArgs pa{};
    pa.x = zb;
    pa.pre = kPreNone;
    pa.na = 1;
    pa.normw[0] = proj_of(c, L.proj[5]).d.normw;
    pa.normwT[0] = proj_of(c, L.proj[5]).d.normwT;
    pa.eps = m.cfg.rms_norm_eps;
    pa.qs = m.qs;
    tbeg(c, kRkPrologue);
    MMF_HIP(launch_prologue(mode, pa, act, st));
    tend(c);
    GemmArgs ga = gemm_args(c, &L.proj[5], 1, rows, mode, m.frac);
    ga.epi = kEpiAdd;
    ga.add = resid;
    ga.out[0] = h;
    tbeg(c, kRkGemmDown);
    proj_gemm(c, m, ga, act, st, l, 5);
    tend(c);
  }
}

// Final norm + lm_head over rows (hgrn_model.cpp:235,245,440-441) -> logits [rows, V].
void lm_rows(mmf_ctx* c, Model& m, int rows, const float* h, float* logits) {
  const Mode mode = static_cast<Mode>(m.mode);
  RowScratch& s = m.rs;
  const Geom& g = proj_of(c, m.lm).d.g;
  ActBuf act = make_act(s.acty, s.actq, s.actct, s.actsa, mode, g, rows, 1);
  PrologueArgs pa{};
  pa.x = h;
  pa.pre = kPreNorm;
  pa.pre_w = m.norm_w;
  pa.pre_wT = m.norm_wT;
  pa.na = 1;
  pa.normw[0] = proj_of(c, m.lm).d.normw;
  pa.normwT[0] = proj_of(c, m.lm).d.normwT;
  pa.eps = m.cfg.rms_norm_eps;
  pa.qs = m.qs;
  tbeg(c, kRkLM);
  MMF_HIP(launch_prologue(mode, pa, act, c->stream));
  tend(c);
  GemmArgs ga = gemm_args(c, &m.lm, 1, rows, mode, m.frac);
  ga.out[0] = logits;
  tbeg(c, kRkLM);
  proj_gemm(c, m, ga, act, c->stream, -1, 6);
  tend(c);
}

int lm_grid(const Model& m) {
  const int g = static_cast<int>((m.cfg.vocab_size + kGroup - 1) / kGroup);
  return lm_blocks(g, static_cast<int>(m.cfg.hidden_size));
}

DecArgs dec_base(Model& m) {
  DecArgs a{};
  a.H = static_cast<int>(m.cfg.hidden_size);
  a.I = static_cast<int>(m.cfg.intermediate_size);
  a.vocab = static_cast<int>(m.cfg.vocab_size);
  a.eps = m.cfg.rms_norm_eps;
  a.qs = m.qs;
  a.embT = static_cast<const float*>(m.embT.p);
  a.oLc = m.gH.Lc;
  a.oK8 = m.gH.K8;
  a.keys = static_cast<unsigned long long*>(m.key.p);
  a.nkeys = lm_grid(m);
  return a;
}

void set_proj(mmf_ctx* c, Model& m, DecArgs& a, int slot, int id) {
  a.p[slot] = proj_of(c, id).d;
  a.inv_fixed[slot] = inv_fixed_of(a.p[slot].scale_w, m.frac);
}

// Single-row lm_head on the chain-transposed device row x: logits (may be null) and, if
// want_key, the argmax key (atomicMax into a cleared key).
void lm_single(mmf_ctx* c, Model& m, const float* x, float* logits, bool want_key) {
  DecArgs a = dec_base(m);
  set_proj(c, m, a, 0, m.lm);
  a.x = x;
  a.pre_w = m.norm_wT;
  a.out = logits;
  if (!want_key) a.keys = nullptr;
  tbeg(c, kRkLM);
  MMF_HIP(launch_decode(kLM, static_cast<Mode>(m.mode), a, c->stream));
  tend(c);
}

// One kernel of the single-row decode step for stream 0. `full` = part of a real step:
// layer 0 then gathers the embedding row of the argmax key (recording it in the token
// history) and its kO clears the key for this step's lm_head. Timing runs use full =
// false (layer 0 reads h like the others).
void decode_one(mmf_ctx* c, Model& m, DecKind kind, size_t l, bool full = false) {
  const Mode mode = static_cast<Mode>(m.mode);
  const size_t H = m.cfg.hidden_size;
  float* h = static_cast<float*>(m.h.p);
  float* resid = static_cast<float*>(m.resid.p);
  float* g = static_cast<float*>(m.g.p);
  float* recur = static_cast<float*>(m.recur.p);
  float* z = static_cast<float*>(m.z.p);
  float* state = static_cast<float*>(m.state.p);
  if (kind == kLM) {
    lm_single(c, m, h, nullptr, true);
    return;
  }
  const LayerDev& L = m.layers[l];
  DecArgs a = dec_base(m);
  a.layer = static_cast<int>(l);
  switch (kind) {
    case kIFG:
      for (int k = 0; k < 3; ++k) set_proj(c, m, a, k, L.proj[k]);
      a.x = (l == 0 && full) ? nullptr : h;
      if (a.x == nullptr) {
        a.out = h;  // layer 0: the embedding row becomes h
        a.hist = m.hist.as<int64_t>(1);
        a.hist_pos = m.hist_pos.as<int32_t>(1);
        a.hist_cap = static_cast<int>(m.hist_cap);
      }
      a.pre_w = L.attnT;
      a.lb = L.lb;
      a.state = state + l * H;
      a.recur = recur;
      a.gout = g;
      break;
    case kO:
      set_proj(c, m, a, 0, L.proj[3]);
      a.x = g;
      a.x2 = recur;
      a.pre_w = L.gnT;
      a.hin = h;
      a.out = resid;
      break;
    case kGate:
      set_proj(c, m, a, 0, L.proj[4]);
      a.x = resid;
      a.pre_w = L.mlpT;
      a.out = z;
      a.oLc = m.gI.Lc;  // z is I long
      a.oK8 = m.gI.K8;
      break;
    default:  // kDown
      set_proj(c, m, a, 0, L.proj[5]);
      a.x = z;
      a.hin = resid;
      a.out = h;
      break;
  }
  // each fused launch is one BitLinear group (with its norms and epilogue): timed as matmul
  tbeg(c, kind == kIFG ? kRkGemmIFG : kind == kO ? kRkGemmO : kind == kGate ? kRkGemmGate : kRkGemmDown);
  MMF_HIP(launch_decode(kind, mode, a, c->stream));
  tend(c);
}

void decode_launches(mmf_ctx* c, Model& m) {
  for (size_t l = 0; l < m.layers.size(); ++l)
    for (DecKind k : {kIFG, kO, kGate, kDown}) decode_one(c, m, k, l, true);
  decode_one(c, m, kLM, 0, true);
}

// HIP graphs for the launch-bound loops (MMF_GRAPH=0 turns them off, e.g. under a profiler
// that cannot follow graph launches).
bool graphs_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("MMF_GRAPH");
    return !(e && std::strcmp(e, "0") == 0);
  }();
  return on;
}

// Capture the launches that f() enqueues on the context's stream into an executable graph;
// nullptr if capture or instantiation fails (the caller then launches directly).
template <class F>
hipGraphExec_t capture_graph(mmf_ctx* c, F&& f) {
  hipGraphExec_t exec = nullptr;
  hipGraph_t gr = nullptr;
  if (hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal) == hipSuccess) {
    bool ok = true;
    try {
      f();
    } catch (const Err&) {
      ok = false;
    }
    if (hipStreamEndCapture(c->stream, &gr) != hipSuccess) ok = false;
    if (ok && gr && hipGraphInstantiate(&exec, gr, nullptr, nullptr, 0) != hipSuccess) exec = nullptr;
    if (gr) (void)hipGraphDestroy(gr);
  }
  (void)hipGetLastError();
  return exec;
}

void decode_step(mmf_ctx* c, Model& m) {
  if (c->timer.on) {  // profiling: launch by launch, each between its own events
    decode_launches(c, m);
    return;
  }
  if (graphs_enabled() && !m.graph_tried) {
    m.graph_tried = true;
    m.graph = capture_graph(c, [&] { decode_launches(c, m); });
  }
  if (m.graph) {
    MMF_HIP(hipGraphLaunch(m.graph, c->stream));
  } else {
    decode_launches(c, m);
  }
}

void drop_graph(Model& m) {
  if (m.graph) (void)hipGraphExecDestroy(m.graph);
  m.graph = nullptr;
  m.graph_tried = false;
  if (m.step_graph) (void)hipGraphExecDestroy(m.step_graph);
  m.step_graph = nullptr;
  m.step_B = 0;
}

void reset_state(mmf_ctx* c, Model& m, size_t B) {
  const size_t n = m.cfg.num_hidden_layers * B * m.cfg.hidden_size;
  void* old = m.state.p;
  m.state.as<float>(n);
  if (m.state.p != old) drop_graph(m);  // the graph holds the state pointer
  MMF_HIP(hipMemsetAsync(m.state.p, 0, n * sizeof(float), c->stream));
  m.streams = B;
}

// Prefill T ids of stream b (time scan) and leave the final hidden rows in rs.h.
float* prefill_rows(mmf_ctx* c, Model& m, size_t b, const int64_t* ids, size_t T, float* trace_h,
                    float* trace_state, float* trace_int) {
  check_ids(m, ids, T);
  const size_t H = m.cfg.hidden_size, L = m.cfg.num_hidden_layers, B = m.streams;
  RowScratch& s = m.rs;
  int64_t* dids = s.ids.as<int64_t>(T);
  MMF_HIP(hipMemcpyAsync(dids, ids, T * sizeof(int64_t), hipMemcpyHostToDevice, c->stream));
  float* h = s.h.as<float>(T * H);
  tbeg(c, kRkOther);
  MMF_HIP(launch_embed(m.emb, dids, h, static_cast<int>(T), static_cast<int>(H), c->stream));
  tend(c);
  float* tint = nullptr;
  DBuf tbuf;
  if (trace_int) tint = tbuf.as<float>(5 * T * H);
  for (size_t l = 0; l < L; ++l) {
    float* st = static_cast<float*>(m.state.p) + (l * B + b) * H;
    layer_rows(c, m, static_cast<int>(l), static_cast<int>(T), h, st, false, tint);
    if (trace_h)
      MMF_HIP(hipMemcpyAsync(trace_h + l * T * H, h, T * H * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    if (trace_state)
      MMF_HIP(hipMemcpyAsync(trace_state + l * H, st, H * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    if (trace_int) {
      MMF_HIP(hipMemcpyAsync(trace_int + l * 5 * T * H, tint, 5 * T * H * sizeof(float), hipMemcpyDeviceToHost,
                             c->stream));
      MMF_HIP(hipStreamSynchronize(c->stream));
    }
  }
  if (trace_int || trace_h || trace_state) MMF_HIP(hipStreamSynchronize(c->stream));
  tbuf.release();
  return h;
}

// Whether the prompts of several streams may be stacked into one row range: every elementwise
// SIMD call of the reference then covers whole groups of 8 in each stream (T * H and T * I
// elements), so no element is a tail element and stacking changes no rounding.
bool stackable(const Model& m) { return m.cfg.hidden_size % 8 == 0 && m.cfg.intermediate_size % 8 == 0; }

// Prefill the prompts of streams 0..n-1 (ids concatenated, lens[b] each) as one stack of
// rows: the prologues and GEMMs of every layer run over all prompt rows at once and the
// recurrence scans each stream's segment from its own state. The last row of each stream
// -> final norm + lm_head -> logits [n, V] (device), as a per-stream prefill computes them.
float* prefill_stacked(mmf_ctx* c, Model& m, size_t n, const int64_t* ids, const size_t* lens) {
  const size_t H = m.cfg.hidden_size, L = m.cfg.num_hidden_layers, B = m.streams, V = m.cfg.vocab_size;
  std::vector<int> seg(2 * n + 1);
  size_t R = 0;
  for (size_t b = 0; b < n; ++b) {
    if (lens[b] == 0) fail(MMF_ERR_ARG, "empty prompt");
    seg[b] = static_cast<int>(R);
    R += lens[b];
    seg[n + 1 + b] = static_cast<int>(R - 1);
  }
  if (R * H > static_cast<size_t>(INT32_MAX)) fail(MMF_ERR_ARG, "prompts too long");
  seg[n] = static_cast<int>(R);
  check_ids(m, ids, R);
  RowScratch& s = m.rs;
  int64_t* dids = s.ids.as<int64_t>(R);
  int* dseg = s.segs.as<int>(seg.size());
  MMF_HIP(hipMemcpyAsync(dids, ids, R * sizeof(int64_t), hipMemcpyHostToDevice, c->stream));
  MMF_HIP(hipMemcpyAsync(dseg, seg.data(), seg.size() * sizeof(int), hipMemcpyHostToDevice, c->stream));
  float* h = s.h.as<float>(R * H);
  MMF_HIP(launch_embed(m.emb, dids, h, static_cast<int>(R), static_cast<int>(H), c->stream));
  for (size_t l = 0; l < L; ++l)
    layer_rows(c, m, static_cast<int>(l), static_cast<int>(R), h, static_cast<float*>(m.state.p) + l * B * H, false,
               nullptr, dseg, static_cast<int>(n));
  float* last = s.resid.as<float>(n * H);  // free once the layers are done
  MMF_HIP(launch_gather_rows(h, dseg + n + 1, last, static_cast<int>(n), static_cast<int>(H), c->stream));
  float* lg = s.logits.as<float>(n * V);
  lm_rows(c, m, static_cast<int>(n), last, lg);
  return lg;
}

// The token of the last lm_head: the max over its per-block argmax keys.
int64_t read_key(mmf_ctx* c, Model& m) {
  const int n = lm_grid(m);
  std::vector<unsigned long long> k(n);
  MMF_HIP(hipMemcpyAsync(k.data(), m.key.p, n * sizeof(unsigned long long), hipMemcpyDeviceToHost, c->stream));
  MMF_HIP(hipStreamSynchronize(c->stream));
  unsigned long long best = 0;
  for (auto v : k) best = v > best ? v : best;
  return key_index(best);
}

void clear_key(mmf_ctx* c, Model& m) {
  MMF_HIP(hipMemsetAsync(m.key.p, 0, kLMBlocks * sizeof(unsigned long long), c->stream));
  MMF_HIP(hipMemsetAsync(m.hist_pos.p, 0, sizeof(int32_t), c->stream));
}

// Greedy B=1 decode on the row kernels, one launch sequence per token (the path while an
// external matmul is set: it runs on the host, which the captured single-row decode graph
// cannot call). hlast: the prompt's last hidden row; appends the generated ids to out.
void generate_rows(mmf_ctx* c, Model& m, const float* hlast, size_t new_tokens, int64_t eos_id, int64_t* out,
                   size_t& len, mmf_token_cb cb, void* user) {
  const size_t H = m.cfg.hidden_size, V = m.cfg.vocab_size;
  RowScratch& s = m.rs;
  float* lg = s.logits.as<float>(V);
  int64_t* am = s.am.as<int64_t>(1);
  int64_t* d = s.ids.as<int64_t>(1);
  auto head = [&](const float* x) {
    lm_rows(c, m, 1, x, lg);
    MMF_HIP(launch_argmax_rows(lg, 1, static_cast<int>(V), am, c->stream));
    int64_t t = 0;
    MMF_HIP(hipMemcpyAsync(&t, am, sizeof(int64_t), hipMemcpyDeviceToHost, c->stream));
    MMF_HIP(hipStreamSynchronize(c->stream));
    return t;
  };
  int64_t t = head(hlast);
  for (size_t k = 0; k < new_tokens; ++k) {
    if (k > 0) {
      MMF_HIP(hipMemcpyAsync(d, &t, sizeof(int64_t), hipMemcpyHostToDevice, c->stream));
      float* h = s.h.as<float>(H);
      tbeg(c, kRkOther);
      MMF_HIP(launch_embed(m.emb, d, h, 1, static_cast<int>(H), c->stream));
      tend(c);
      for (size_t l = 0; l < m.cfg.num_hidden_layers; ++l)
        layer_rows(c, m, static_cast<int>(l), 1, h, static_cast<float*>(m.state.p) + l * H, true, nullptr);
      t = head(h);
    }
    out[len++] = t;
    if (cb) cb(user, t);
    if (t == eos_id) break;
  }
}

}  // namespace

// =========================================================================================
// C ABI
// =========================================================================================
extern "C" {

// Scratch of mmf_bitlinear_noalloc. Each GPU holds its own copy at its own address; host
// code never passes the array's name to a kernel (on the host it is only a stand-in for the
// symbol): it uses the device address that hipGetSymbolAddress returned for that GPU.
static __device__ __align__(256) unsigned char scratch[MMF_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};  // device address of `scratch` per device, once resolved

// Resolves the device address of `scratch` on `device`, which must be current. Called by
// mmf_create once per device.
hipError_t resolve_scratch(int device) {
  if (device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_dev[device]) return hipSuccess;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if (!p) return hipErrorInvalidSymbol;
  g_scratch_dev[device] = p;
  return hipSuccess;
}
}  // namespace

int mmf_create(mmf_ctx** out, int device) {
  if (!out) return MMF_ERR_ARG;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= device || device < 0) {
    g_create_err = "no HIP device " + std::to_string(device);
    return MMF_ERR_NODEV;
  }
  hipDeviceProp_t prop{};
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
    g_create_err = "hipGetDeviceProperties failed";
    return MMF_ERR_NODEV;
  }
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    g_create_err = std::string("device is ") + prop.gcnArchName + ", this build targets gfx950";
    return MMF_ERR_NODEV;
  }
  auto* c = new (std::nothrow) mmf_ctx;
  if (!c) return MMF_ERR_ARG;
  c->device = device;
  c->prop = prop;
  if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
    g_create_err = "stream creation failed";
    delete c;
    return MMF_ERR_HIP;
  }
  const hipError_t se = resolve_scratch(device);
  if (se != hipSuccess) {
    g_create_err = std::string("device address of the no-alloc scratch: ") + hipGetErrorString(se);
    (void)hipStreamDestroy(c->stream);
    delete c;
    return MMF_ERR_HIP;
  }
  *out = c;
  return MMF_OK;
}

void mmf_destroy(mmf_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  drop_graph(c->model);
  for (auto& p : c->projs) {
    if (p.mem) (void)hipFree(p.mem);
    if (p.mem4) (void)hipFree(p.mem4);
  }
  for (auto& kv : c->model.tensors)
    if (kv.second.p) (void)hipFree(kv.second.p);
  Model& m = c->model;
  for (DBuf* b : {&m.h, &m.resid, &m.g, &m.recur, &m.z, &m.logits, &m.key, &m.hist, &m.hist_pos, &m.state, &m.embT,
                  &m.normT, &m.ext_codes, &m.ext_acc})
    b->release();
  RowScratch& s = m.rs;
  for (DBuf* b : {&s.ids, &s.h, &s.resid, &s.i, &s.f, &s.g, &s.recur, &s.scan, &s.z, &s.logits, &s.state0, &s.am,
                  &s.acty, &s.actq, &s.actct, &s.actsa, &s.segs, &s.chunk})
    b->release();
  for (DBuf* b : {&c->raw, &c->opy, &c->opq, &c->opct, &c->opsa, &c->opstate, &c->gws, &c->hmx, &c->hmacc})
    b->release();
  c->pin_x.release();
  c->pin_acc.release();
  (void)hipStreamDestroy(c->stream);
  delete c;
}

const char* mmf_last_error(const mmf_ctx* c) { return c ? c->err.c_str() : g_create_err.c_str(); }

int mmf_sync(mmf_ctx* c) {
  return guard(c, [&] { MMF_HIP(hipStreamSynchronize(c->stream)); });
}

void* mmf_stream(mmf_ctx* c) { return c ? static_cast<void*>(c->stream) : nullptr; }

int mmf_device_info(mmf_ctx* c, char* name, size_t cap, int* cus) {
  return guard(c, [&] {
    if (name && cap) {
      std::snprintf(name, cap, "%s (%s)", c->prop.name, c->prop.gcnArchName);
    }
    if (cus) *cus = c->prop.multiProcessorCount;
  });
}

int mmf_malloc(mmf_ctx* c, void** dev, size_t bytes) {
  return guard(c, [&] {
    if (!dev) fail(MMF_ERR_ARG, "null out pointer");
    MMF_HIP(hipMalloc(dev, bytes ? bytes : 1));
  });
}

int mmf_free(mmf_ctx* c, void* dev) {
  return guard(c, [&] { MMF_HIP(hipFree(dev)); });
}

int mmf_upload(mmf_ctx* c, void* dev, const void* host, size_t bytes) {
  return guard(c, [&] {
    MMF_HIP(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, c->stream));
    MMF_HIP(hipStreamSynchronize(c->stream));
  });
}

int mmf_download(mmf_ctx* c, void* host, const void* dev, size_t bytes) {
  return guard(c, [&] {
    MMF_HIP(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, c->stream));
    MMF_HIP(hipStreamSynchronize(c->stream));
  });
}

int mmf_proj_register(mmf_ctx* c, const int8_t* wq, size_t N, size_t K, float scale_w, const float* normw,
                      int* proj_id) {
  return guard(c, [&] {
    if (!wq || !proj_id) fail(MMF_ERR_ARG, "null argument");
    void* raw = c->raw.get(N * K);
    MMF_HIP(hipMemcpyAsync(raw, wq, N * K, hipMemcpyHostToDevice, c->stream));
    *proj_id = register_proj(c, static_cast<const int8_t*>(raw), N, K, scale_w, normw, nullptr);
  });
}

int mmf_proj_update(mmf_ctx* c, int id, const int8_t* wq) {
  return guard(c, [&] {
    if (!wq) fail(MMF_ERR_ARG, "null argument");
    const Proj& P = proj_of(c, id);
    const Geom& g = P.d.g;
    const size_t NK = static_cast<size_t>(g.N) * g.K;
    void* raw = c->raw.get(NK);
    MMF_HIP(hipMemcpyAsync(raw, wq, NK, hipMemcpyHostToDevice, c->stream));
    const hipError_t e = launch_pack(static_cast<const int8_t*>(raw), g, const_cast<uint32_t*>(P.d.pk),
                                     const_cast<int8_t*>(P.d.tail), const_cast<int32_t*>(P.d.rowsum), c->stream);
    if (e == hipErrorInvalidValue) fail(MMF_ERR_ARG, "projection weights must be ternary (-1, 0, +1)");
    MMF_HIP(e);
    MMF_HIP(launch_pack_mfma(P.d.pk, g, P.d.pair != 0, const_cast<uint32_t*>(P.d.pkm), c->stream));
    if (P.d.pk4) MMF_HIP(launch_pack4(P.d.pk, g, const_cast<uint32_t*>(P.d.pk4), c->stream));
  });
}

int mmf_proj_shape(mmf_ctx* c, int id, size_t* N, size_t* K) {
  return guard(c, [&] {
    const Proj& p = proj_of(c, id);
    if (N) *N = p.d.g.N;
    if (K) *K = p.d.g.K;
  });
}

int mmf_proj_release(mmf_ctx* c, int id) {
  return guard(c, [&] {
    (void)proj_of(c, id);
    for (const auto& kv : c->model.tensors)
      if (kv.second.proj == id) fail(MMF_ERR_STATE, "proj_id " + std::to_string(id) + " belongs to the loaded model");
    MMF_HIP(hipStreamSynchronize(c->stream));
    Proj& P = c->projs[id];
    MMF_HIP(hipFree(P.mem));
    if (P.mem4) MMF_HIP(hipFree(P.mem4));
    P = Proj{};
  });
}

int mmf_ternary_matmul_host(mmf_ctx* c, int k, const int* ids, const int32_t* const* x, int32_t* const* acc,
                            size_t b) {
  return guard(c, [&] {
    if (k < 1 || k > 64 || !ids || !x || !acc) fail(MMF_ERR_ARG, "invalid arguments");
    if (b == 0) return;
    if (b > (1u << 24)) fail(MMF_ERR_ARG, "too many rows");
    size_t xo[64], ao[64], in = 0, out = 0;
    for (int z = 0; z < k; ++z) {
      const Proj& p = proj_of(c, ids[z]);
      if (!x[z] || !acc[z]) fail(MMF_ERR_ARG, "null buffer");
      xo[z] = in;
      ao[z] = out;
      in += b * static_cast<size_t>(p.d.g.K);
      out += b * static_cast<size_t>(p.d.g.N);
    }
    int32_t* hx = c->pin_x.as<int32_t>(in);
    int32_t* ha = c->pin_acc.as<int32_t>(out);
    int32_t* dx = c->hmx.as<int32_t>(in);
    int32_t* da = c->hmacc.as<int32_t>(out);
    for (int z = 0; z < k; ++z) std::memcpy(hx + xo[z], x[z], b * proj_of(c, ids[z]).d.g.K * sizeof(int32_t));
    // few rows of projections of one shape (a decode step's i/f/g cluster, o, gate, down,
    // lm_head): one kernel for all k that reads the codes from the pinned staging and writes the
    // accumulators straight into it (no copy engine round trips)
    const Geom& g0 = proj_of(c, ids[0]).d.g;
    bool one_shape = static_cast<int>(b) <= seam_max_rows() && k <= kSeamMaxProj;
    for (int z = 1; z < k && one_shape; ++z) {
      const Geom& gz = proj_of(c, ids[z]).d.g;
      one_shape = gz.N == g0.N && gz.K == g0.K;
    }
    if (one_shape) {
      (void)dx;
      SeamArgs sa{};
      for (int z = 0; z < k; ++z) {
        sa.pk[z] = proj_of(c, ids[z]).d.pk;
        sa.tail[z] = proj_of(c, ids[z]).d.tail;
        sa.rowsum[z] = proj_of(c, ids[z]).d.rowsum;
      }
      sa.x = hx;
      sa.acc = ha;
      sa.g = g0;
      sa.b = static_cast<int>(b);
      MMF_HIP(launch_seam_dot(sa, k, c->stream));
      MMF_HIP(hipStreamSynchronize(c->stream));
      for (int z = 0; z < k; ++z) std::memcpy(acc[z], ha + ao[z], b * static_cast<size_t>(g0.N) * sizeof(int32_t));
      return;
    }
    MMF_HIP(hipMemcpyAsync(dx, hx, in * sizeof(int32_t), hipMemcpyHostToDevice, c->stream));
    for (int z = 0; z < k; ++z) {
      const Proj& p = proj_of(c, ids[z]);
      ActBuf act = make_act(c->opy, c->opq, c->opct, c->opsa, kFixed, p.d.g, static_cast<int>(b), 1);
      MMF_HIP(launch_codes_to_planes(dx + xo[z], act, c->stream));
      GemmArgs ga = gemm_args(c, &ids[z], 1, static_cast<int>(b), kFixed, 10);
      ga.raw_acc = true;
      ga.acc[0] = da + ao[z];
      run_gemm(c, ga, act, c->stream);
    }
    MMF_HIP(hipMemcpyAsync(ha, da, out * sizeof(int32_t), hipMemcpyDeviceToHost, c->stream));
    MMF_HIP(hipStreamSynchronize(c->stream));
    for (int z = 0; z < k; ++z) std::memcpy(acc[z], ha + ao[z], b * proj_of(c, ids[z]).d.g.N * sizeof(int32_t));
  });
}

int mmf_ternary_matmul(mmf_ctx* c, int id, const int32_t* x, int32_t* acc, size_t b) {
  return guard(c, [&] {
    if (b == 0) return;
    const Proj& p = proj_of(c, id);
    ActBuf act = make_act(c->opy, c->opq, c->opct, c->opsa, kFixed, p.d.g, static_cast<int>(b), 1);
    MMF_HIP(launch_codes_to_planes(x, act, c->stream));
    GemmArgs ga = gemm_args(c, &id, 1, static_cast<int>(b), kFixed, 10);
    ga.raw_acc = true;
    ga.acc[0] = acc;
    run_gemm(c, ga, act, c->stream);
  });
}

// A fixed device region that one call carves its scratch from (mmf_bitlinear_noalloc).
struct FixedScratch {
  char* base;
  size_t cap;
};

// MMF_OPFUSE=0: single-row BitLinear calls take the two-launch path too (comparisons).
static bool fused_op_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("MMF_OPFUSE");
    return !(e && e[0] == '0');
  }();
  return on;
}

// fs == nullptr: the activations and the split-K partials live in the context's grow-only
// buffers; otherwise in fs, and nothing is allocated (sizes beyond fs->cap are refused
// before any launch).
static void bitlinear_impl(mmf_ctx* c, const int* ids, int k, int mode, int frac, float eps, const float* x,
                           float* const* outs, size_t rows, int32_t* acc, const FixedScratch* fs = nullptr) {
  if (k < 1 || k > 3) fail(MMF_ERR_ARG, "cluster size must be 1..3");
  if (mode < 0 || mode > 2) fail(MMF_ERR_ARG, "invalid mode");
  if (frac < 0 || frac > 30) fail(MMF_ERR_ARG, "invalid frac_bits");
  if (rows == 0) return;
  if (rows > (1u << 24)) fail(MMF_ERR_ARG, "too many rows");
  if (!x) fail(MMF_ERR_ARG, "null input");
  for (int z = 0; z < k; ++z)
    if (!outs[z]) fail(MMF_ERR_ARG, "null output");
  const Proj& p0 = proj_of(c, ids[0]);
  for (int z = 0; z < k; ++z) {
    const Proj& p = proj_of(c, ids[z]);
    if (p.d.g.N != p0.d.g.N || p.d.g.K != p0.d.g.K) fail(MMF_ERR_ARG, "cluster projections differ in shape");
    if (!p.d.normw) fail(MMF_ERR_ARG, "projection registered without a norm weight");
  }
  const Mode md = static_cast<Mode>(mode);
  // one row of one projection: norm, encoding and GEMV in one launch (the batch-1 decode
  // kernel's operator kind), where it applies (integer modes, model widths, aligned row)
  if (rows == 1 && k == 1 && fused_op_enabled() && (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
    DecArgs d{};
    d.p[0] = p0.d;
    d.inv_fixed[0] = inv_fixed_of(p0.d.scale_w, frac);
    d.eps = eps;
    d.qs = static_cast<float>(1u << frac);
    d.x = x;
    d.out = outs[0];
    d.acc = acc;
    tbeg(c, kRkGemmIFG);
    const hipError_t e = launch_decode(kOp, md, d, c->stream);
    tend(c);
    if (e != hipErrorNotSupported) {
      MMF_HIP(e);
      return;
    }
  }
  GemmArgs ga = gemm_args(c, ids, k, static_cast<int>(rows), md, frac);
  for (int z = 0; z < k; ++z) ga.out[z] = outs[z];
  ga.acc[0] = acc;
  const size_t wsb = gemm_workspace_bytes(ga);
  ActBuf act;
  if (!fs) {
    act = make_act(c->opy, c->opq, c->opct, c->opsa, md, p0.d.g, static_cast<int>(rows), k);
    ga.ws = wsb ? static_cast<int32_t*>(c->gws.get(wsb)) : nullptr;
  } else {
    act = act_shape(p0.d.g, static_cast<int>(rows), k);
    size_t b[5];
    act_bytes(md, act, b);
    b[4] = wsb;
    size_t off[5], end = 0;
    for (int i = 0; i < 5; ++i) {
      off[i] = end;
      end = (end + b[i] + 255) / 256 * 256;
    }
    if (end > fs->cap)
      fail(MMF_ERR_ARG, "bitlinear needs " + std::to_string(end) + " bytes of scratch for " + std::to_string(rows) +
                            " rows of this projection, more than the " + std::to_string(fs->cap) +
                            " bytes of the static scratch: split the rows over several calls");
    act.y = b[0] ? reinterpret_cast<float*>(fs->base + off[0]) : nullptr;
    act.q = b[1] ? reinterpret_cast<int8_t*>(fs->base + off[1]) : nullptr;
    act.ct = b[2] ? reinterpret_cast<int32_t*>(fs->base + off[2]) : nullptr;
    act.sa = b[3] ? reinterpret_cast<float*>(fs->base + off[3]) : nullptr;
    ga.ws = wsb ? reinterpret_cast<int32_t*>(fs->base + off[4]) : nullptr;
  }
  PrologueArgs pa{};
  pa.x = x;
  pa.pre = kPreNone;
  pa.na = k;
  for (int z = 0; z < k; ++z) {
    pa.normw[z] = proj_of(c, ids[z]).d.normw;
    pa.normwT[z] = proj_of(c, ids[z]).d.normwT;
  }
  pa.eps = eps;
  pa.qs = static_cast<float>(1u << frac);
  tbeg(c, kRkPrologue);
  MMF_HIP(launch_prologue(md, pa, act, c->stream));
  tend(c);
  tbeg(c, kRkGemmIFG);
  MMF_HIP(launch_gemm(ga, act, c->stream));
  tend(c);
}

extern "C++" {
// Runs f() `reps` times with the row timer on and adds each kind's average microseconds
// per run to kind_us[kRkCount].
template <class F>
void time_kinds(mmf_ctx* c, int reps, F&& f, double* kind_us) {
  RowTimer& t = c->timer;
  t.used = 0;
  t.kinds.clear();
  t.on = true;
  try {
    for (int r = 0; r < reps; ++r) f();
  } catch (...) {
    t.on = false;
    throw;
  }
  t.on = false;
  MMF_HIP(hipStreamSynchronize(c->stream));
  for (int k = 0; k < kRkCount; ++k) kind_us[k] = 0.0;
  for (size_t i = 0; i < t.kinds.size(); ++i) {
    float ms = 0.0f;
    MMF_HIP(hipEventElapsedTime(&ms, t.pool[2 * i], t.pool[2 * i + 1]));
    kind_us[t.kinds[i]] += 1000.0 * ms / reps;
  }
}

// Average microseconds per run of f() over `reps` runs after `warmup`, one event pair
// around the whole batch of runs.
template <class F>
double time_runs(mmf_ctx* c, int warmup, int reps, F&& f) {
  for (int i = 0; i < warmup; ++i) f();
  hipEvent_t e0, e1;
  MMF_HIP(hipEventCreate(&e0));
  MMF_HIP(hipEventCreate(&e1));
  float ms = 0.0f;
  hipError_t err = hipEventRecord(e0, c->stream);
  if (err == hipSuccess) {
    for (int i = 0; i < reps; ++i) f();
    err = hipEventRecord(e1, c->stream);
  }
  if (err == hipSuccess) err = hipEventSynchronize(e1);
  if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  MMF_HIP(err);
  return 1000.0 * ms / reps;
}

// Average microseconds per run of f() when `reps` runs are captured back to back in one
// HIP graph (device time without the host's per-launch cost); time_runs() if graphs are
// off or the capture fails. f() must allocate nothing once it has run (warmup >= 1).
template <class F>
double time_graph_runs(mmf_ctx* c, int warmup, int reps, F&& f) {
  if (warmup < 1) warmup = 1;
  for (int i = 0; i < warmup; ++i) f();
  hipGraphExec_t ge = graphs_enabled() ? capture_graph(c, [&] {
    for (int i = 0; i < reps; ++i) f();
  }) : nullptr;
  if (!ge) return time_runs(c, 0, reps, f);
  hipEvent_t e0 = nullptr, e1 = nullptr;
  float ms = 0.0f;
  hipError_t err = hipGraphLaunch(ge, c->stream);  // first replay uploads the graph
  if (err == hipSuccess) err = hipEventCreate(&e0);
  if (err == hipSuccess) err = hipEventCreate(&e1);
  if (err == hipSuccess) err = hipEventRecord(e0, c->stream);
  if (err == hipSuccess) err = hipGraphLaunch(ge, c->stream);
  if (err == hipSuccess) err = hipEventRecord(e1, c->stream);
  if (err == hipSuccess) err = hipEventSynchronize(e1);
  if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  (void)hipGraphExecDestroy(ge);
  MMF_HIP(err);
  return 1000.0 * ms / reps;
}
}  // extern "C++"

int mmf_bitlinear(mmf_ctx* c, int id, int mode, int frac, float eps, const float* x, float* out, size_t rows,
                  int32_t* acc) {
  return guard(c, [&] { bitlinear_impl(c, &id, 1, mode, frac, eps, x, &out, rows, acc); });
}

int mmf_bitlinear_noalloc(mmf_ctx* c, int id, int mode, int frac, float eps, const float* x, float* out,
                          size_t rows, int32_t* acc) {
  return guard(c, [&] {
    void* p = nullptr;
    {
      std::lock_guard<std::mutex> lk(g_scratch_mu);
      p = c->device < kMaxDevices ? g_scratch_dev[c->device] : nullptr;
    }
    if (!p) fail(MMF_ERR_STATE, "no-alloc scratch not resolved on this device");
    const FixedScratch fs{static_cast<char*>(p), MMF_NOALLOC_SCRATCH_BYTES};
    bitlinear_impl(c, &id, 1, mode, frac, eps, x, &out, rows, acc, &fs);
  });
}

int mmf_workspace_bytes(mmf_ctx* c, size_t* bytes) {
  return guard(c, [&] {
    if (!bytes) fail(MMF_ERR_ARG, "null output");
    size_t n = 0;
    for (const DBuf* b : {&c->opy, &c->opq, &c->opct, &c->opsa, &c->opstate, &c->gws}) n += b->n;
    *bytes = n;
  });
}

int mmf_bitlinear_cluster(mmf_ctx* c, const int* ids, int k, int mode, int frac, float eps, const float* x,
                          float* const* outs, size_t rows) {
  return guard(c, [&] {
    if (!ids || !outs) fail(MMF_ERR_ARG, "null argument");
    bitlinear_impl(c, ids, k, mode, frac, eps, x, outs, rows, nullptr);
  });
}

int mmf_bitlinear_codes(mmf_ctx* c, const float* x, const float* normw, int32_t* codes, size_t rows, size_t K,
                        float eps, int frac) {
  return guard(c, [&] {
    if (frac < 0 || frac > 30) fail(MMF_ERR_ARG, "invalid frac_bits");
    if (!rows || !K) return;
    float* y = c->opy.as<float>(rows * K);
    MMF_HIP(launch_rmsnorm(x, normw, y, static_cast<int>(rows), static_cast<int>(K), eps, c->stream));
    MMF_HIP(launch_quant_rows(y, codes, static_cast<int>(rows), static_cast<int>(K), static_cast<float>(1u << frac),
                              c->stream));
  });
}

int mmf_rmsnorm(mmf_ctx* c, float* y, const float* x, const float* w, size_t rows, size_t cols, float eps) {
  return guard(c, [&] {
    if (rows && cols) MMF_HIP(launch_rmsnorm(x, w, y, static_cast<int>(rows), static_cast<int>(cols), eps, c->stream));
  });
}

int mmf_swiglu(mmf_ctx* c, float* out, const float* a, const float* b, size_t n) {
  return guard(c, [&] {
    if (n) MMF_HIP(launch_swiglu(a, b, out, n, c->stream));
  });
}

int mmf_hgrn_scan(mmf_ctx* c, float* out, const float* i, const float* f, size_t T, size_t D, float* state) {
  return guard(c, [&] {
    if (T && D) MMF_HIP(launch_scan(i, f, out, state, static_cast<int>(T), static_cast<int>(D), c->stream));
  });
}

int mmf_rmsnorm_swishgate(mmf_ctx* c, float* out, const float* g, const float* o, const float* w, size_t rows,
                          size_t cols, float eps) {
  return guard(c, [&] {
    if (rows && cols)
      MMF_HIP(launch_swishgate(g, o, w, out, static_cast<int>(rows), static_cast<int>(cols), eps, c->stream));
  });
}

// ---- model ------------------------------------------------------------------------------
int mmf_model_begin(mmf_ctx* c, const mmf_config* cfg) {
  return guard(c, [&] {
    if (!cfg || !cfg->vocab_size || !cfg->hidden_size || !cfg->num_hidden_layers || !cfg->intermediate_size)
      fail(MMF_ERR_ARG, "invalid config");
    if (c->model.begun) fail(MMF_ERR_STATE, "a model was already begun on this context");
    c->model.cfg = *cfg;
    c->model.begun = true;
  });
}

int mmf_model_tensor(mmf_ctx* c, const char* name, int dtype, const size_t* shape, int ndim, const void* data) {
  return guard(c, [&] {
    Model& m = c->model;
    if (!m.begun || m.finalized) fail(MMF_ERR_STATE, "mmf_model_tensor outside begin/finalize");
    if (!name || !data || ndim < 0 || ndim > 4 || (dtype != 0 && dtype != 1)) fail(MMF_ERR_ARG, "invalid tensor");
    DevTensor t;
    t.dtype = dtype;
    t.shape.assign(shape, shape + ndim);
    const size_t bytes = t.numel() * (dtype == 0 ? 4 : 1);
    const std::string nm(name);
    const bool is_wq = nm.size() > 3 && nm.compare(nm.size() - 3, 3, ".wq") == 0;
    if (is_wq) {
      if (dtype != 1 || ndim != 2) fail(MMF_ERR_ARG, "weights: " + nm + " must be a 2-D i8 tensor");
      void* raw = c->raw.get(bytes);
      MMF_HIP(hipMemcpyAsync(raw, data, bytes, hipMemcpyHostToDevice, c->stream));
      t.proj = register_proj(c, static_cast<const int8_t*>(raw), t.shape[0], t.shape[1], 1.0f, nullptr, nullptr);
    } else {
      MMF_HIP(hipMalloc(&t.p, bytes ? bytes : 1));
      MMF_HIP(hipMemcpyAsync(t.p, data, bytes, hipMemcpyHostToDevice, c->stream));
      MMF_HIP(hipStreamSynchronize(c->stream));
      if (dtype == 0 && t.numel() <= 16) {
        t.host_small.resize(t.numel());
        std::memcpy(t.host_small.data(), data, bytes);
      }
    }
    auto it = m.tensors.find(nm);
    if (it != m.tensors.end()) {
      if (it->second.p) (void)hipFree(it->second.p);
      m.tensors.erase(it);
    }
    m.tensors.emplace(nm, std::move(t));
  });
}

int mmf_model_finalize(mmf_ctx* c, int mode, int frac) {
  return guard(c, [&] {
    Model& m = c->model;
    if (!m.begun) fail(MMF_ERR_STATE, "mmf_model_begin first");
    if (mode < 0 || mode > 2) fail(MMF_ERR_ARG, "invalid mode");
    if (frac < 0 || frac > 30) fail(MMF_ERR_ARG, "invalid frac_bits");
    const size_t V = m.cfg.vocab_size, H = m.cfg.hidden_size, L = m.cfg.num_hidden_layers,
                 I = m.cfg.intermediate_size;
    if (I % 16 != 0) fail(MMF_ERR_ARG, "intermediate_size must be a multiple of 16");
    auto f32 = [&](const std::string& n, std::vector<size_t> shape) -> const float* {
      const DevTensor& t = tensor_of(m, n);
      if (t.dtype != 0) fail(MMF_ERR_ARG, "weights: " + n + " must be f32");
      check_shape(t, n, shape);
      return static_cast<const float*>(t.p);
    };
    auto proj = [&](const std::string& tag, size_t N, size_t K) -> int {
      const DevTensor& w = tensor_of(m, tag + ".wq");
      check_shape(w, tag + ".wq", {N, K});
      const DevTensor& sw = tensor_of(m, tag + ".scale_w");
      if (sw.host_small.size() != 1) fail(MMF_ERR_ARG, "weights: " + tag + ".scale_w must hold one f32");
      Proj& p = c->projs[w.proj];
      p.d.scale_w = sw.host_small[0];
      p.d.inv_scale_w = 1.0f / p.d.scale_w;
      p.d.inv_fixed = inv_fixed_of(p.d.scale_w, frac);
      p.d.normw = f32(tag + ".normw", {K});
      return w.proj;
    };
    m.emb = f32("model.embeddings", {V, H});
    m.norm_w = f32("model.norm.w", {H});
    m.lm = proj("lm_head", V, H);
    const float* lb = nullptr;
    if (m.cfg.use_lower_bound) lb = f32("lower_bounds", {L, H});
    m.layers.assign(L, LayerDev{});
    static const char* names[6] = {"i_proj", "f_proj", "g_proj", "o_proj", "gate_proj", "down_proj"};
    for (size_t l = 0; l < L; ++l) {
      const std::string p = "model.layers." + std::to_string(l);
      LayerDev& Ld = m.layers[l];
      Ld.attn = f32(p + ".attn_norm.w", {H});
      Ld.mlp = f32(p + ".mlp_norm.w", {H});
      Ld.gn = f32(p + ".g_norm.w", {H});
      for (int j = 0; j < 6; ++j) {
        const size_t N = j == 4 ? 2 * I : H, K = j == 5 ? I : H;
        Ld.proj[j] = proj(p + "." + names[j], N, K);
      }
      // the gate matrix feeds swiglu(gate, up): interleave its halves in the tile order
      ProjDev& gd = c->projs[Ld.proj[4]].d;
      if (!gd.pair && pkm_pairable(gd.g)) {
        MMF_HIP(launch_pack_mfma(gd.pk, gd.g, true, const_cast<uint32_t*>(gd.pkm), c->stream));
        gd.pair = 1;
      }
      Ld.lb = (lb && l > 0) ? lb + l * H : nullptr;  // hgrn_model.cpp:116-117
    }
    // chain-transposed copies for the single-row decode kernels
    m.gH = make_geom(static_cast<int>(H), static_cast<int>(H));
    m.gI = make_geom(static_cast<int>(H), static_cast<int>(I));
    const size_t WH = chain_len(m.gH), WI = chain_len(m.gI);
    float* et = m.embT.as<float>(V * WH);
    MMF_HIP(launch_to_chain(m.emb, et, static_cast<int>(V), static_cast<int>(H), m.gH.Lc, c->stream));
    const size_t nvec = 2 + L * 8;  // final norm, lm normw; per layer 3 norms + 5 H-long normw (+ down)
    float* nt = m.normT.as<float>(nvec * WH + L * WI);
    size_t off = 0;
    auto tr = [&](const float* src, bool ilong) -> const float* {
      float* dst = nt + off;
      off += ilong ? WI : WH;
      MMF_HIP(launch_to_chain(src, dst, 1, static_cast<int>(ilong ? I : H), ilong ? m.gI.Lc : m.gH.Lc, c->stream));
      return dst;
    };
    m.norm_wT = tr(m.norm_w, false);
    c->projs[m.lm].d.normwT = tr(c->projs[m.lm].d.normw, false);
    for (size_t l = 0; l < L; ++l) {
      LayerDev& Ld = m.layers[l];
      Ld.attnT = tr(Ld.attn, false);
      Ld.mlpT = tr(Ld.mlp, false);
      Ld.gnT = tr(Ld.gn, false);
      for (int j = 0; j < 6; ++j) c->projs[Ld.proj[j]].d.normwT = tr(c->projs[Ld.proj[j]].d.normw, j == 5);
    }
    if (mode == kFloat)  // the batch-1 float GEMVs of i/f/g, o and down read fp4 codes
      for (size_t l = 0; l < L; ++l)
        for (int j : {0, 1, 2, 3, 5}) ensure_pk4(c, c->projs[m.layers[l].proj[j]]);
    m.mode = mode;
    m.frac = frac;
    m.qs = static_cast<float>(1u << frac);
    alloc_decode(c, m);
    m.finalized = true;
    drop_graph(m);
    reset_state(c, m, 1);
    MMF_HIP(hipStreamSynchronize(c->stream));
  });
}

int mmf_model_config(mmf_ctx* c, mmf_config* cfg) {
  return guard(c, [&] {
    if (!cfg) fail(MMF_ERR_ARG, "null cfg");
    *cfg = c->model.cfg;
  });
}

int mmf_model_generate(mmf_ctx* c, const int64_t* ids, size_t n, size_t new_tokens, int64_t eos_id, int64_t* out,
                       size_t cap, size_t* out_len, mmf_token_cb cb, void* user) {
  return guard(c, [&] {
    Model& m = model_of(c);
    if (!ids || n == 0) fail(MMF_ERR_ARG, "empty prompt");
    if (!out || cap < n + new_tokens) fail(MMF_ERR_ARG, "output capacity below prompt + new_tokens");
    std::memcpy(out, ids, n * sizeof(int64_t));
    size_t len = n;
    reset_state(c, m, 1);  // hgrn_model.cpp:315
    if (new_tokens + 1 > m.hist_cap) {
      m.hist.as<int64_t>(new_tokens + 1);
      m.hist_cap = new_tokens + 1;
      drop_graph(m);
    }
    clear_key(c, m);
    float* h = prefill_rows(c, m, 0, ids, n, nullptr, nullptr, nullptr);
    if (new_tokens == 0) {
      if (out_len) *out_len = len;
      return;
    }
    if (m.ext_on()) {  // the external matmul runs on the host: one row step at a time
      generate_rows(c, m, h + (n - 1) * m.cfg.hidden_size, new_tokens, eos_id, out, len, cb, user);
      if (out_len) *out_len = len;
      return;
    }
    MMF_HIP(launch_to_chain(h + (n - 1) * m.cfg.hidden_size, static_cast<float*>(m.h.p), 1,
                            static_cast<int>(m.cfg.hidden_size), m.gH.Lc, c->stream));
    lm_single(c, m, static_cast<float*>(m.h.p), nullptr, true);
    int64_t t = read_key(c, m);
    out[len++] = t;
    if (cb) cb(user, t);
    if (t == eos_id) {
      if (out_len) *out_len = len;
      return;
    }
    const size_t rest = new_tokens - 1;
    if (eos_id < 0) {
      // no stop condition: run ahead in chunks, report tokens after each chunk
      const size_t chunk = cb ? 16 : rest;
      size_t done = 0;
      std::vector<int64_t> hv;
      while (done < rest) {
        const size_t k = std::min(chunk, rest - done);
        for (size_t s = 0; s < k; ++s) decode_step(c, m);
        done += k;
        // hist[0..done) = tokens consumed by the steps; the last produced one is in key
        hv.resize(done);
        MMF_HIP(hipMemcpyAsync(hv.data(), m.hist.p, done * sizeof(int64_t), hipMemcpyDeviceToHost, c->stream));
        const int64_t last = read_key(c, m);
        for (size_t s = len - n; s < done; ++s) {
          out[len++] = hv[s];
          if (cb) cb(user, hv[s]);
        }
        (void)last;
        if (done == rest) {
          out[len++] = last;
          if (cb) cb(user, last);
        }
      }
    } else {
      for (size_t s = 0; s < rest; ++s) {
        decode_step(c, m);
        t = read_key(c, m);
        out[len++] = t;
        if (cb) cb(user, t);
        if (t == eos_id) break;
      }
    }
    if (out_len) *out_len = len;
  });
}

int mmf_model_reset(mmf_ctx* c, size_t streams) {
  return guard(c, [&] {
    Model& m = model_of(c);
    if (streams == 0) fail(MMF_ERR_ARG, "streams must be >= 1");
    reset_state(c, m, streams);
    if (m.hist_cap == 0) {
      m.hist.as<int64_t>(1);
      m.hist_cap = 1;
    }
    clear_key(c, m);
  });
}

static void deliver_rows(mmf_ctx* c, Model& m, const float* logits_dev, size_t rows, float* logits, int64_t* argmax) {
  const size_t V = m.cfg.vocab_size;
  if (logits)
    MMF_HIP(hipMemcpyAsync(logits, logits_dev, rows * V * sizeof(float), hipMemcpyDeviceToHost, c->stream));
  if (argmax) {
    int64_t* d = m.rs.am.as<int64_t>(rows);
    MMF_HIP(launch_argmax_rows(logits_dev, static_cast<int>(rows), static_cast<int>(V), d, c->stream));
    MMF_HIP(hipMemcpyAsync(argmax, d, rows * sizeof(int64_t), hipMemcpyDeviceToHost, c->stream));
  }
  MMF_HIP(hipStreamSynchronize(c->stream));
}

int mmf_model_prefill(mmf_ctx* c, size_t stream, const int64_t* ids, size_t n, float* logits, int64_t* argmax) {
  return guard(c, [&] {
    Model& m = model_of(c);
    if (stream >= m.streams) fail(MMF_ERR_ARG, "stream index beyond mmf_model_reset's count");
    if (!ids || n == 0) fail(MMF_ERR_ARG, "empty prompt");
    float* h = prefill_rows(c, m, stream, ids, n, nullptr, nullptr, nullptr);
    float* lg = m.logits.as<float>(m.cfg.vocab_size);
    MMF_HIP(launch_to_chain(h + (n - 1) * m.cfg.hidden_size, static_cast<float*>(m.h.p), 1,
                            static_cast<int>(m.cfg.hidden_size), m.gH.Lc, c->stream));
    lm_single(c, m, static_cast<float*>(m.h.p), lg, false);
    deliver_rows(c, m, lg, 1, logits, argmax);
  });
}

int mmf_model_prefill_streams(mmf_ctx* c, size_t n, const int64_t* ids, const size_t* lens, float* logits,
                              int64_t* argmax) {
  return guard(c, [&] {
    Model& m = model_of(c);
    if (n == 0 || n > m.streams) fail(MMF_ERR_ARG, "stream count beyond mmf_model_reset's count");
    if (!ids || !lens) fail(MMF_ERR_ARG, "null prompts");
    const size_t V = m.cfg.vocab_size, H = m.cfg.hidden_size;
    if (stackable(m)) {
      float* lg = prefill_stacked(c, m, n, ids, lens);
      deliver_rows(c, m, lg, n, logits, argmax);
      return;
    }
    size_t at = 0;  // one stream at a time (a stack would move SIMD tail elements)
    for (size_t b = 0; b < n; ++b) {
      if (lens[b] == 0) fail(MMF_ERR_ARG, "empty prompt");
      float* h = prefill_rows(c, m, b, ids + at, lens[b], nullptr, nullptr, nullptr);
      float* lg = m.logits.as<float>(V);
      MMF_HIP(launch_to_chain(h + (lens[b] - 1) * H, static_cast<float*>(m.h.p), 1, static_cast<int>(H), m.gH.Lc,
                              c->stream));
      lm_single(c, m, static_cast<float*>(m.h.p), lg, false);
      deliver_rows(c, m, lg, 1, logits ? logits + b * V : nullptr, argmax ? argmax + b : nullptr);
      at += lens[b];
    }
  });
}

}  // extern "C"

namespace {

// The launches of one lockstep serving step of the m.streams streams: embedding of the
// device tokens d, every layer over the B rows, final norm + lm_head into lg, argmax into am.
void step_kernels(mmf_ctx* c, Model& m, const int64_t* d, float* h, float* lg, int64_t* am) {
  const size_t B = m.streams, H = m.cfg.hidden_size, V = m.cfg.vocab_size;
  tbeg(c, kRkOther);
  MMF_HIP(launch_embed(m.emb, d, h, static_cast<int>(B), static_cast<int>(H), c->stream));
  tend(c);
  for (size_t l = 0; l < m.cfg.num_hidden_layers; ++l)
    layer_rows(c, m, static_cast<int>(l), static_cast<int>(B), h, static_cast<float*>(m.state.p) + l * B * H, true,
               nullptr);
  lm_rows(c, m, static_cast<int>(B), h, lg);
  tbeg(c, kRkLM);
  MMF_HIP(launch_argmax_rows(lg, static_cast<int>(B), static_cast<int>(V), am, c->stream));
  tend(c);
}

}  // namespace

extern "C" {

int mmf_model_step(mmf_ctx* c, const int64_t* tokens, float* logits, int64_t* argmax) {
  return guard(c, [&] {
    Model& m = model_of(c);
    const size_t B = m.streams, H = m.cfg.hidden_size, V = m.cfg.vocab_size;
    if (!tokens) fail(MMF_ERR_ARG, "null tokens");
    check_ids(m, tokens, B);
    RowScratch& s = m.rs;
    int64_t* d = s.ids.as<int64_t>(B);
    MMF_HIP(hipMemcpyAsync(d, tokens, B * sizeof(int64_t), hipMemcpyHostToDevice, c->stream));
    float* h = s.h.as<float>(B * H);
    float* lg = s.logits.as<float>(B * V);
    int64_t* am = s.am.as<int64_t>(B);
    // embedding, all layers, final norm + lm_head, argmax: captured once per stream count
    // and replayed while no scratch buffer has moved (the first step runs them directly)
    auto work = [&] { step_kernels(c, m, d, h, lg, am); };
    if (m.ext_on() || c->timer.on) {  // host matmul or per-launch profiling: no graph
      work();
    } else if (m.step_graph && m.step_B == B && m.step_epoch == dbuf_epoch.load()) {
      MMF_HIP(hipGraphLaunch(m.step_graph, c->stream));
    } else {
      work();
      if (m.step_graph) (void)hipGraphExecDestroy(m.step_graph);
      m.step_graph = nullptr;
      if (graphs_enabled()) {
        const uint64_t ep = dbuf_epoch.load();
        hipGraphExec_t g = capture_graph(c, work);
        if (g && dbuf_epoch.load() == ep) {
          m.step_graph = g;
          m.step_B = B;
          m.step_epoch = ep;
        } else if (g) {
          (void)hipGraphExecDestroy(g);
        }
      }
    }
    if (logits) MMF_HIP(hipMemcpyAsync(logits, lg, B * V * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    if (argmax) MMF_HIP(hipMemcpyAsync(argmax, am, B * sizeof(int64_t), hipMemcpyDeviceToHost, c->stream));
    MMF_HIP(hipStreamSynchronize(c->stream));
  });
}

int mmf_model_profile(mmf_ctx* c, int on) {
  return guard(c, [&] {
    RowTimer& t = c->timer;
    if (on && !t.on) {
      t.used = 0;
      t.kinds.clear();
    }
    t.on = on != 0;
  });
}

int mmf_model_profile_read(mmf_ctx* c, double* us, uint64_t* launches) {
  return guard(c, [&] {
    RowTimer& t = c->timer;
    double acc[MMF_PROF_KINDS] = {};
    uint64_t n[MMF_PROF_KINDS] = {};
    if (!t.kinds.empty()) {
      MMF_HIP(hipStreamSynchronize(c->stream));
      for (size_t i = 0; i < t.kinds.size(); ++i) {
        float ms = 0.0f;
        MMF_HIP(hipEventElapsedTime(&ms, t.pool[2 * i], t.pool[2 * i + 1]));
        const int k = t.kinds[i];
        const int op = k == kRkPrologue ? MMF_PROF_NORM
                       : k == kRkMixer  ? MMF_PROF_MIXER
                       : k == kRkLM     ? MMF_PROF_LM_HEAD
                       : k == kRkOther  ? MMF_PROF_EMBED
                                        : MMF_PROF_MATMUL;
        acc[op] += 1000.0 * ms;
        ++n[op];
      }
    }
    t.used = 0;
    t.kinds.clear();
    for (int k = 0; k < MMF_PROF_KINDS; ++k) {
      if (us) us[k] = acc[k];
      if (launches) launches[k] = n[k];
    }
  });
}

int mmf_model_set_matmul(mmf_ctx* c, mmf_matmul_fn fn, void* user) {
  return guard(c, [&] {
    Model& m = model_of(c);
    m.ext_fn = fn;
    m.ext_user = fn ? user : nullptr;
  });
}

int mmf_model_set_scan(mmf_ctx* c, int chunked) {
  return guard(c, [&] {
    if (chunked != 0 && chunked != 1) fail(MMF_ERR_ARG, "mmf_model_set_scan: chunked must be 0 or 1");
    Model& m = model_of(c);
    m.chunked_scan = chunked != 0;
  });
}

int mmf_model_state(mmf_ctx* c, float* out) {
  return guard(c, [&] {
    Model& m = model_of(c);
    const size_t n = m.cfg.num_hidden_layers * m.streams * m.cfg.hidden_size;
    MMF_HIP(hipMemcpyAsync(out, m.state.p, n * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    MMF_HIP(hipStreamSynchronize(c->stream));
  });
}

int mmf_model_forward(mmf_ctx* c, const int64_t* ids, size_t T, float* logits) {
  return guard(c, [&] {
    Model& m = model_of(c);
    if (!ids || T == 0 || !logits) fail(MMF_ERR_ARG, "invalid forward arguments");
    check_ids(m, ids, T);
    const size_t H = m.cfg.hidden_size, V = m.cfg.vocab_size;
    RowScratch& s = m.rs;
    int64_t* d = s.ids.as<int64_t>(T);
    MMF_HIP(hipMemcpyAsync(d, ids, T * sizeof(int64_t), hipMemcpyHostToDevice, c->stream));
    float* h = s.h.as<float>(T * H);
    MMF_HIP(launch_embed(m.emb, d, h, static_cast<int>(T), static_cast<int>(H), c->stream));
    float* st = s.state0.as<float>(H);
    for (size_t l = 0; l < m.cfg.num_hidden_layers; ++l) {
      MMF_HIP(hipMemsetAsync(st, 0, H * sizeof(float), c->stream));  // fresh state (hgrn_model.cpp:233)
      layer_rows(c, m, static_cast<int>(l), static_cast<int>(T), h, st, false, nullptr);
    }
    float* lg = s.logits.as<float>(T * V);
    lm_rows(c, m, static_cast<int>(T), h, lg);
    MMF_HIP(hipMemcpyAsync(logits, lg, T * V * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    MMF_HIP(hipStreamSynchronize(c->stream));
  });
}

int mmf_model_trace(mmf_ctx* c, const int64_t* ids, size_t T, float* h, float* state, float* internals) {
  return guard(c, [&] {
    Model& m = model_of(c);
    if (!ids || T == 0 || !h || !state) fail(MMF_ERR_ARG, "invalid trace arguments");
    reset_state(c, m, 1);
    prefill_rows(c, m, 0, ids, T, h, state, internals);
  });
}

int mmf_model_time_decode(mmf_ctx* c, int warmup, int reps, double* step_us, double* kind_us) {
  return guard(c, [&] {
    Model& m = model_of(c);
    if (reps < 1 || warmup < 0) fail(MMF_ERR_ARG, "invalid reps");
    if (m.ext_on()) fail(MMF_ERR_STATE, "timing runs the built-in kernels: clear the external matmul first");
    if (c->timer.on) fail(MMF_ERR_STATE, "timing while the op profile is on");
    if (m.streams != 1) reset_state(c, m, 1);
    if (m.hist_cap < static_cast<size_t>(warmup + reps) + 1) {
      m.hist.as<int64_t>(warmup + reps + 1);
      m.hist_cap = warmup + reps + 1;
      drop_graph(m);
    }
    clear_key(c, m);
    MMF_HIP(hipMemsetAsync(m.hist_pos.p, 0, sizeof(int32_t), c->stream));
    hipEvent_t e0, e1;
    MMF_HIP(hipEventCreate(&e0));
    MMF_HIP(hipEventCreate(&e1));
    for (int i = 0; i < warmup; ++i) decode_step(c, m);
    MMF_HIP(hipEventRecord(e0, c->stream));
    for (int i = 0; i < reps; ++i) decode_step(c, m);
    MMF_HIP(hipEventRecord(e1, c->stream));
    MMF_HIP(hipEventSynchronize(e1));
    float ms = 0.0f;
    MMF_HIP(hipEventElapsedTime(&ms, e0, e1));
    if (step_us) *step_us = 1000.0 * ms / reps;
    if (kind_us) {
      // Per kind: the kernels of that kind for all layers, back to back, `reps` times. With
      // graphs the launches are captured and replayed, so the average per launch is the
      // kernel's execution time plus the graph's launch gap; without graphs every kernel
      // records an event pair at its own start and end (what a profiler's kernel trace reads).
      const size_t L = m.layers.size();
      for (int k = 0; k < 5; ++k) {
        const size_t nl = (k == 4) ? 1 : L;
        const int per = std::max(1, std::min(reps, static_cast<int>(512 / nl)));
        auto launches = [&] {
          for (int r = 0; r < per; ++r)
            for (size_t l = 0; l < nl; ++l) decode_one(c, m, static_cast<DecKind>(k), l);
        };
        hipGraphExec_t gx = graphs_enabled() ? capture_graph(c, launches) : nullptr;
        if (gx) {
          const int rounds = std::max(1, reps / per);
          hipError_t err = hipGraphLaunch(gx, c->stream);  // warm-up replay
          if (err == hipSuccess) err = hipEventRecord(e0, c->stream);
          for (int r = 0; r < rounds && err == hipSuccess; ++r) err = hipGraphLaunch(gx, c->stream);
          if (err == hipSuccess) err = hipEventRecord(e1, c->stream);
          if (err == hipSuccess) err = hipEventSynchronize(e1);
          if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
          (void)hipGraphExecDestroy(gx);
          MMF_HIP(err);
          kind_us[k] = 1000.0 * ms / (static_cast<double>(rounds) * per * nl);
          continue;
        }
        std::vector<hipEvent_t> ev(2 * nl);
        for (auto& e : ev) MMF_HIP(hipEventCreate(&e));
        double total = 0.0;
        for (int r = 0; r < reps + 1; ++r) {
          for (size_t l = 0; l < nl; ++l) {
            g_launch_events = LaunchEvents{ev[2 * l], ev[2 * l + 1]};
            try {
              decode_one(c, m, static_cast<DecKind>(k), l);
            } catch (...) {
              g_launch_events = LaunchEvents{};
              throw;
            }
            g_launch_events = LaunchEvents{};
          }
          MMF_HIP(hipEventSynchronize(ev[2 * nl - 1]));
          if (r == 0) continue;  // warm-up pass
          for (size_t l = 0; l < nl; ++l) {
            MMF_HIP(hipEventElapsedTime(&ms, ev[2 * l], ev[2 * l + 1]));
            total += ms;
          }
        }
        for (auto& e : ev) (void)hipEventDestroy(e);
        kind_us[k] = 1000.0 * total / (static_cast<double>(reps) * nl);
      }
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
  });
}

int mmf_time_bitlinear(mmf_ctx* c, int id, int mode, int frac, float eps, const float* x, float* out, size_t rows,
                       int warmup, int reps, double* total_us, double* prologue_us, double* gemm_us) {
  return guard(c, [&] {
    if (reps < 1 || warmup < 0 || rows == 0) fail(MMF_ERR_ARG, "invalid reps/rows");
    if (c->timer.on) fail(MMF_ERR_STATE, "timing while the op profile is on");
    auto f = [&] { bitlinear_impl(c, &id, 1, mode, frac, eps, x, &out, rows, nullptr); };
    const double t = time_graph_runs(c, warmup, reps, f);
    if (total_us) *total_us = t;
    if (prologue_us || gemm_us) {
      double k[kRkCount];
      time_kinds(c, reps, f, k);
      if (prologue_us) *prologue_us = k[kRkPrologue];
      if (gemm_us) *gemm_us = k[kRkGemmIFG];
    }
  });
}

int mmf_measure_peaks(mmf_ctx* c, double* out4) {
  return guard(c, [&] {
    if (!out4) fail(MMF_ERR_ARG, "null output");
    int dev = 0, cus = 0;
    MMF_HIP(hipGetDevice(&dev));
    MMF_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    MMF_HIP(measure_peaks(cus, c->stream, out4));
  });
}

int mmf_model_time_step(mmf_ctx* c, const int64_t* tokens, int warmup, int reps, double* kind_us) {
  return guard(c, [&] {
    Model& m = model_of(c);
    if (!tokens || !kind_us || reps < 1 || warmup < 0) fail(MMF_ERR_ARG, "invalid tokens/reps");
    if (m.ext_on()) fail(MMF_ERR_STATE, "timing runs the built-in kernels: clear the external matmul first");
    if (c->timer.on) fail(MMF_ERR_STATE, "timing while the op profile is on");
    const size_t B = m.streams, H = m.cfg.hidden_size, V = m.cfg.vocab_size;
    check_ids(m, tokens, B);
    RowScratch& s = m.rs;
    int64_t* d = s.ids.as<int64_t>(B);
    MMF_HIP(hipMemcpyAsync(d, tokens, B * sizeof(int64_t), hipMemcpyHostToDevice, c->stream));
    float* h = s.h.as<float>(B * H);
    float* lg = s.logits.as<float>(B * V);
    int64_t* am = s.am.as<int64_t>(B);
    auto f = [&] { step_kernels(c, m, d, h, lg, am); };
    for (int i = 0; i < warmup; ++i) f();
    time_kinds(c, reps, f, kind_us);
  });
}

int mmf_model_time_prefill(mmf_ctx* c, const int64_t* ids, size_t T, int warmup, int reps, double* total_us,
                           double* kind_us) {
  return guard(c, [&] {
    Model& m = model_of(c);
    if (!ids || T == 0 || reps < 1 || warmup < 0) fail(MMF_ERR_ARG, "invalid prompt/reps");
    if (m.ext_on()) fail(MMF_ERR_STATE, "timing runs the built-in kernels: clear the external matmul first");
    if (c->timer.on) fail(MMF_ERR_STATE, "timing while the op profile is on");
    if (m.streams != 1) reset_state(c, m, 1);
    const int H = static_cast<int>(m.cfg.hidden_size);
    auto f = [&] {
      float* h = prefill_rows(c, m, 0, ids, T, nullptr, nullptr, nullptr);
      tbeg(c, kRkLM);
      MMF_HIP(launch_to_chain(h + (T - 1) * static_cast<size_t>(H), static_cast<float*>(m.h.p), 1, H, m.gH.Lc,
                              c->stream));
      tend(c);
      lm_single(c, m, static_cast<float*>(m.h.p), nullptr, true);  // timed as kRkLM inside
    };
    const double t = time_runs(c, warmup, reps, f);
    if (total_us) *total_us = t;
    if (kind_us) time_kinds(c, reps, f, kind_us);
  });
}

}  // extern "C"
