// runtime.hip -- the C ABI of libtgohip: context, weight upload and repack,
// KV pool, the batched step (Batch.step, batch.go:314-458), the op-level entry
// points, and the Scheduler (scheduler.go) driving it.
#include "common.h"
#include "host/hostlogic.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <deque>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

extern uint16_t tgohip_f16_bits(float x, int* saturated);

namespace tgohip {

static thread_local std::string g_err;
void set_error(const std::string& m) { g_err = m; }
int fail(int code, const std::string& m) {
  g_err = m;
  return code;
}
std::string hip_message(hipError_t e, const char* what) {
  return std::string("hip: ") + what + ": " + hipGetErrorString(e);
}

constexpr size_t kBufAlign = (size_t)2 << 20;

// The allocation-free linear's split-K workspace: a static device array, one
// copy per GPU the library runs on, held until the process ends. Host code
// never passes `scratch` itself (its host-side name is not a device address):
// tgohip_open looks up each device's address once with hipGetSymbolAddress
// and every launch takes that address.
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices] = {};

// With `device` current: its address of `scratch`, looked up on first use.
int scratch_setup(int device, void** out) {
  if (device < 0 || device >= kMaxDevices)
    return fail(TGOHIP_EDEVICE, "scratch: device " + std::to_string(device) + " beyond the table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(TGOHIP_EDEVICE, hip_message(e, "hipGetSymbolAddress(scratch)"));
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return 0;
}

// Grow-only device buffer.
struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
  int ensure(size_t n) {
    if (n <= bytes) return 0;
    // Whole 2 MiB pages: each buffer starts on its own page. With sizes as
    // asked, the step's attention ran 4% slower or not depending on how the
    // buffers happened to fall (one process or the other); rounded, it
    // always runs the faster way.
    n = (n + kBufAlign - 1) / kBufAlign * kBufAlign;
    // a step still in flight may read the old buffer (the scheduler's
    // overlap mode): let the device drain before it goes
    if (p) (void)hipDeviceSynchronize();
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
    hipError_t e = hipMalloc(&p, n);
    if (e != hipSuccess) {
      p = nullptr;
      return fail(TGOHIP_ENOMEM, "device allocation of " + std::to_string(n) + " bytes: " +
                                     hipGetErrorString(e));
    }
    bytes = n;
    // TGOHIP_DEBUG_NAN_FILL=1: every activation and workspace buffer starts as
    // all-ones bytes (NaN in f32 and f16), so a kernel that reads memory no
    // earlier kernel wrote shows up as NaN logits or changed tokens.
    static const bool nan_fill = [] {
      const char* v = getenv("TGOHIP_DEBUG_NAN_FILL");
      return v && atoi(v) != 0;
    }();
    if (nan_fill) {
      e = hipMemset(p, 0xff, n);
      if (e == hipSuccess) e = hipDeviceSynchronize();
      if (e != hipSuccess) return fail(TGOHIP_EDEVICE, hip_message(e, "debug fill"));
    }
    return 0;
  }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
};

// Sub-ports of a layer's fused projections, one bit each once uploaded.
enum { SUB_WQ = 1, SUB_WK = 2, SUB_WV = 4, SUB_WGATE = 8, SUB_WUP = 16, SUB_ALL = 31 };

struct Layer {
  PackedWeight qkv, wo, gateup, down;
  int bound = 0;  // SUB_* bits of the fused QKV and gate/up sub-ports written
  float* g_attn = nullptr;
  float* g_ffn = nullptr;
  float* g_q = nullptr;
  float* g_k = nullptr;
};

}  // namespace tgohip

using namespace tgohip;

struct tgohip_ctx {
  int device = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;
  int ncu = 256;
  bool configured = false;
  tgohip_model_cfg cfg{};
  std::vector<Layer> layers;
  void* embed = nullptr;
  uint16_t* embed_scales = nullptr;
  int embed_form = -1;
  PackedWeight lm_head;
  float* g_final = nullptr;
  double* inv_freq = nullptr;
  half_t* kc = nullptr;
  half_t* vc = nullptr;
  int kv_positions = 0;
  int precision = 1;  // 1 (default): tgo's f32 arithmetic (hi+lo pairs), 0: f16 operands
  int cascade = 0;    // minimum sequences sharing a prefix for prefix-shared attention (0: off)
  // activations and workspaces
  DevBuf h, xn, qkv, q, attn, act, lastn, logits, argmax, margin, meta, gemm_ws, part_o, part_ml;
  DevBuf amax_part;  // per-chunk partials of the greedy selection
  DevBuf rows;  // [2][rows]: positions and slots derived on the device
  DevBuf rope;  // [rows][32] float4: the rows' rotary cos and sin (rope_table)
  int rows_cap = 0, batch_cap = 0;
  int last_batch = 0;  // members of the last launched step (its margins are in `margin`)
  // The head of the last launched step ran over the members that worked only:
  // logits row i is member head_rows[i]'s (empty: one row per member).
  std::vector<int32_t> head_rows;
  // pinned staging for per-step metadata
  void* pinned = nullptr;
  size_t pinned_bytes = 0;
  hipEvent_t staged = nullptr;  // the last H2D copy out of `pinned`
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  std::vector<void*> allocs;  // weight and gain allocations owned by the context
  std::map<int, PackedWeight> handles;
  int next_handle = 1;
  // profiling: HIP events around the launches of the kernels in prof_mask
  // (TGOHIP_PROF_* bits) in every prof_stride-th layer of a step
  bool profile = false;
  int prof_stride = 1;
  int prof_mask = 1 << TGOHIP_PROF_ATTN;
  std::vector<hipEvent_t> prof_ev;  // [2 sets][layers][kinds][begin, end]
  double prof_ms[TGOHIP_PROF_KINDS] = {}, prof_bytes[TGOHIP_PROF_KINDS] = {},
         prof_flops[TGOHIP_PROF_KINDS] = {};
  int64_t prof_launches[TGOHIP_PROF_KINDS] = {};
  void* scratch = nullptr;  // this device's address of the static split-K workspace
};

namespace {

int alloc_owned(tgohip_ctx* c, void** p, size_t bytes) {
  hipError_t e = hipMalloc(p, bytes);
  if (e != hipSuccess)
    return fail(TGOHIP_ENOMEM, "device allocation of " + std::to_string(bytes) + " bytes: " +
                                   hipGetErrorString(e));
  c->allocs.push_back(*p);
  return 0;
}

void free_owned(tgohip_ctx* c, void* p) {
  if (!p) return;
  auto it = std::find(c->allocs.begin(), c->allocs.end(), p);
  if (it != c->allocs.end()) c->allocs.erase(it);
  (void)hipFree(p);
}

int ensure_pinned(tgohip_ctx* c, size_t bytes) {
  if (c->staged) TGOHIP_HIP(hipEventSynchronize(c->staged));
  if (bytes <= c->pinned_bytes) return 0;
  if (c->pinned) (void)hipHostFree(c->pinned);
  c->pinned = nullptr;
  c->pinned_bytes = 0;
  TGOHIP_HIP(hipHostMalloc(&c->pinned, bytes, hipHostMallocDefault));
  c->pinned_bytes = bytes;
  return 0;
}

// Metadata packer: appends arrays into the pinned staging buffer at 256-byte
// aligned offsets, then one H2D copy moves all of them into c->meta.
struct Stager {
  std::vector<std::pair<const void*, size_t>> parts;
  std::vector<size_t> offs;
  size_t total = 0;
  size_t add(const void* p, size_t bytes) {
    const size_t o = total;
    parts.push_back({p, bytes});
    offs.push_back(o);
    total += (bytes + 255) / 256 * 256;
    return o;
  }
  int upload(tgohip_ctx* c) {
    if (total == 0) return 0;
    int rc = ensure_pinned(c, total);
    if (rc) return rc;
    rc = c->meta.ensure(total);
    if (rc) return rc;
    for (size_t i = 0; i < parts.size(); i++)
      if (parts[i].second) memcpy((char*)c->pinned + offs[i], parts[i].first, parts[i].second);
    TGOHIP_HIP(hipMemcpyAsync(c->meta.p, c->pinned, total, hipMemcpyHostToDevice, c->stream));
    TGOHIP_HIP(hipEventRecord(c->staged, c->stream));
    return 0;
  }
  template <class T> T* dev(tgohip_ctx* c, size_t off) { return (T*)((char*)c->meta.p + off); }
};

int check_shape(int form, int K, int N, const char* what) {
  if (form < TGOHIP_FORM_F16 || form > TGOHIP_FORM_I4_SYM)
    return fail(TGOHIP_EINVAL, std::string(what) + ": form " + std::to_string(form) +
                                   " is not f16, int8, int4 or the symmetric int4 pack");
  if (K <= 0 || N <= 0 || K % 64 != 0 || N % 32 != 0)
    return fail(TGOHIP_EINVAL, std::string(what) + " is [" + std::to_string(K) + "," +
                                   std::to_string(N) + "]; this library takes K a multiple of 64 "
                                   "and N a multiple of 32");
  if (form == TGOHIP_FORM_I4_TGO && N % 128 != 0)
    return fail(TGOHIP_EINVAL, std::string(what) + ": the int4 triple groups 128 flattened "
                                   "elements and N " + std::to_string(N) +
                                   " is not a multiple of 128, so a group would straddle rows");
  return 0;
}

size_t scale_count(int form, int K, int N) {
  const size_t n = (size_t)K * N;
  switch (form) {
    case TGOHIP_FORM_I8: return (n + 31) / 32;
    case TGOHIP_FORM_I4_TGO: return (n + 127) / 128;
    case TGOHIP_FORM_I4_SYM: return (size_t)(K / 32) * N;
  }
  return 0;
}
size_t plane_bytes(int form, int K, int N) {
  const size_t n = (size_t)K * N;
  switch (form) {
    case TGOHIP_FORM_F16: return n * 2;
    case TGOHIP_FORM_I8: return n;
    case TGOHIP_FORM_I4_TGO: return (n + 7) / 8 * 4;
    case TGOHIP_FORM_I4_SYM: return n / 2;
  }
  return 0;
}

// Allocates w as a packed [K, N] weight of `form`.
// Allocates w as a packed [K, N] weight of `form`. The weight counts as bound
// (form >= 0) only once every buffer is allocated; a failure frees the ones
// that were and leaves w unbound.
int alloc_packed(tgohip_ctx* c, PackedWeight& w, int form, int K, int N) {
  PackedWeight n;
  int rc = alloc_owned(c, &n.wp, packed_payload_bytes(form, K, N));
  const size_t sh = packed_scale_halves(form, K, N);
  if (!rc && sh) rc = alloc_owned(c, (void**)&n.ws, sh * 2);
  if (!rc && form == TGOHIP_FORM_I4_TGO) rc = alloc_owned(c, (void**)&n.wz, sh * 2);
  if (rc) {
    free_owned(c, n.wp);
    free_owned(c, n.ws);
    free_owned(c, n.wz);
    return rc;
  }
  n.form = form;
  n.K = K;
  n.N = N;
  w = n;
  return 0;
}

void free_packed(tgohip_ctx* c, PackedWeight& w) {
  free_owned(c, w.wp);
  free_owned(c, w.ws);
  free_owned(c, w.wz);
  w = PackedWeight();
}

// Canonical (host-layout) weight resident on the device, temporary.
struct Canon {
  void* plane = nullptr;
  uint16_t* scales = nullptr;
  uint16_t* zeros = nullptr;
  ~Canon() {
    if (plane) (void)hipFree(plane);
    if (scales) (void)hipFree(scales);
    if (zeros) (void)hipFree(zeros);
  }
};

int canon_alloc(Canon& cn, int form, int K, int N) {
  TGOHIP_HIP(hipMalloc(&cn.plane, plane_bytes(form, K, N)));
  const size_t sc = scale_count(form, K, N);
  if (sc) TGOHIP_HIP(hipMalloc((void**)&cn.scales, sc * 2));
  if (form == TGOHIP_FORM_I4_TGO) TGOHIP_HIP(hipMalloc((void**)&cn.zeros, sc * 2));
  return 0;
}

struct DevFree {
  void* p;
  ~DevFree() { (void)hipFree(p); }
};

// The canonical form of an f32 host plane, quantized on the device (I8 or
// I4_TGO) into cn: the codes of tgohip_quantize_int8 / _int4, bit for bit.
int canon_quantize(tgohip_ctx* c, Canon& cn, int form, int K, int N, const float* w) {
  if (form != TGOHIP_FORM_I8 && form != TGOHIP_FORM_I4_TGO)
    return fail(TGOHIP_EINVAL, "weight_f32: the device quantizes to I8 or I4_TGO (form " +
                                   std::to_string(form) + "); f16 converts on the host (tgohip_to_f16)");
  if (!w) return fail(TGOHIP_EINVAL, "weight: the plane is missing");
  int rc = canon_alloc(cn, form, K, N);
  if (rc) return rc;
  const size_t n = (size_t)K * N;
  float* dw = nullptr;
  TGOHIP_HIP(hipMalloc((void**)&dw, n * sizeof(float)));
  DevFree hold{dw};
  TGOHIP_HIP(hipMemcpyAsync(dw, w, n * sizeof(float), hipMemcpyHostToDevice, c->stream));
  if (form == TGOHIP_FORM_I8)
    launch_quantize_i8(dw, n, (int8_t*)cn.plane, cn.scales, c->stream);
  else
    launch_quantize_i4tgo(dw, n, (uint32_t*)cn.plane, cn.scales, cn.zeros, c->stream);
  TGOHIP_HIP(hipGetLastError());
  TGOHIP_HIP(hipStreamSynchronize(c->stream));  // the staging plane is freed on return
  return 0;
}

int canon_upload(tgohip_ctx* c, Canon& cn, int form, int K, int N, const void* plane,
                 const void* scales, const void* zeros) {
  int rc = canon_alloc(cn, form, K, N);
  if (rc) return rc;
  if (!plane) return fail(TGOHIP_EINVAL, "weight: the plane is missing");
  TGOHIP_HIP(hipMemcpyAsync(cn.plane, plane, plane_bytes(form, K, N), hipMemcpyHostToDevice, c->stream));
  const size_t sc = scale_count(form, K, N);
  if (sc) {
    if (!scales) return fail(TGOHIP_EINVAL, "weight: a quantized form carries scales");
    TGOHIP_HIP(hipMemcpyAsync(cn.scales, scales, sc * 2, hipMemcpyHostToDevice, c->stream));
  }
  if (form == TGOHIP_FORM_I4_TGO) {
    if (!zeros) return fail(TGOHIP_EINVAL, "weight: the int4 triple carries zeros");
    TGOHIP_HIP(hipMemcpyAsync(cn.zeros, zeros, sc * 2, hipMemcpyHostToDevice, c->stream));
  }
  return 0;
}

// Synthesises a canonical weight on the device (the CPU restatement's
// generator: oracle.c synth_weight).
int canon_synth(tgohip_ctx* c, Canon& cn, uint64_t seed, uint64_t stream, int form, int K, int N,
                double sigma) {
  int rc = canon_alloc(cn, form, K, N);
  if (rc) return rc;
  const size_t n = (size_t)K * N, sc = scale_count(form, K, N);
  hipStream_t st = c->stream;
  switch (form) {
    case TGOHIP_FORM_F16: launch_synth_f16(seed, stream * 4, n, sigma, (uint16_t*)cn.plane, st); break;
    case TGOHIP_FORM_I8:
      launch_synth_i8(seed, stream * 4, n, (int8_t*)cn.plane, st);
      launch_synth_absf16(seed, stream * 4 + 1, sc, sigma / 64.0, cn.scales, st);
      break;
    case TGOHIP_FORM_I4_TGO:
      launch_synth_i4tgo(seed, stream * 4, n, (uint32_t*)cn.plane, st);
      launch_synth_absf16(seed, stream * 4 + 1, sc, sigma / 4.0, cn.scales, st);
      launch_synth_zero(seed, stream * 4 + 2, sc, cn.zeros, st);
      break;
    case TGOHIP_FORM_I4_SYM:
      launch_synth_i4sym(seed, stream * 4, K, N, (uint32_t*)cn.plane, st);
      launch_synth_absf16(seed, stream * 4 + 1, sc, sigma / 4.0, cn.scales, st);
      break;
  }
  TGOHIP_HIP(hipGetLastError());
  return 0;
}

enum PortKind { P_EMBED, P_LMHEAD, P_WQ, P_WK, P_WV, P_WO, P_WGATE, P_WUP, P_WDOWN, P_BAD };

PortKind parse_port(const char* port, int& layer) {
  layer = -1;
  if (!strcmp(port, "embed")) return P_EMBED;
  if (!strcmp(port, "lm_head")) return P_LMHEAD;
  char* end = nullptr;
  const long l = strtol(port, &end, 10);
  if (end == port || *end != '.') return P_BAD;
  layer = (int)l;
  const char* name = end + 1;
  static const std::pair<const char*, PortKind> names[] = {
      {"wq", P_WQ}, {"wk", P_WK}, {"wv", P_WV}, {"wo", P_WO},
      {"wgate", P_WGATE}, {"wup", P_WUP}, {"wdown", P_WDOWN}};
  for (auto& p : names)
    if (!strcmp(name, p.first)) return p.second;
  return P_BAD;
}

// Places one port's canonical device weight into the context's packed layout.
int place_weight(tgohip_ctx* c, PortKind kind, int l, int form, int K, int N, const Canon& cn,
                 const char* port) {
  const tgohip_model_cfg& m = c->cfg;
  const int d = m.hidden, qw = m.heads * m.head_dim, kw = m.kv_heads * m.head_dim, f = m.ffn;
  int wantK = 0, wantN = 0;
  switch (kind) {
    case P_LMHEAD: wantK = d; wantN = m.vocab; break;
    case P_WQ: wantK = d; wantN = qw; break;
    case P_WK: case P_WV: wantK = d; wantN = kw; break;
    case P_WO: wantK = qw; wantN = d; break;
    case P_WGATE: case P_WUP: wantK = d; wantN = f; break;
    case P_WDOWN: wantK = f; wantN = d; break;
    default: break;
  }
  if (K != wantK || N != wantN)
    return fail(TGOHIP_EINVAL, std::string("weight ") + port + " is [" + std::to_string(K) + "," +
                                   std::to_string(N) + "] and the config asks for [" +
                                   std::to_string(wantK) + "," + std::to_string(wantN) + "]");
  int rc = check_shape(form, K, N, port);
  if (rc) return rc;
  PackedWeight* w = nullptr;
  int fusedN = N, stride = 1, off = 0;
  if (kind == P_LMHEAD) {
    w = &c->lm_head;
  } else {
    Layer& L = c->layers[l];
    switch (kind) {
      case P_WQ: w = &L.qkv; fusedN = qw + 2 * kw; off = 0; break;
      case P_WK: w = &L.qkv; fusedN = qw + 2 * kw; off = qw / 32; break;
      case P_WV: w = &L.qkv; fusedN = qw + 2 * kw; off = (qw + kw) / 32; break;
      case P_WO: w = &L.wo; break;
      case P_WGATE: w = &L.gateup; fusedN = 2 * f; stride = 2; off = 0; break;
      case P_WUP: w = &L.gateup; fusedN = 2 * f; stride = 2; off = 1; break;
      case P_WDOWN: w = &L.down; break;
      default: break;
    }
  }
  if (w->form >= 0 && w->form != form) {
    if (fusedN != N)
      return fail(TGOHIP_EINVAL, std::string("weight ") + port + " is form " + std::to_string(form) +
                                     " and the projection it is fused with is form " +
                                     std::to_string(w->form) + "; fused projections share a form");
    free_packed(c, *w);
  }
  if (w->form < 0) {
    rc = alloc_packed(c, *w, form, K, fusedN);
    if (rc) return rc;
    // a fresh fused buffer holds none of its sub-ports yet
    if (kind == P_WQ || kind == P_WK || kind == P_WV) c->layers[l].bound &= ~(SUB_WQ | SUB_WK | SUB_WV);
    if (kind == P_WGATE || kind == P_WUP) c->layers[l].bound &= ~(SUB_WGATE | SUB_WUP);
  }
  rc = repack_enqueue(form, cn.plane, cn.scales, cn.zeros, K, N, *w, stride, off, c->stream);
  if (rc) return rc;
  switch (kind) {
    case P_WQ: c->layers[l].bound |= SUB_WQ; break;
    case P_WK: c->layers[l].bound |= SUB_WK; break;
    case P_WV: c->layers[l].bound |= SUB_WV; break;
    case P_WGATE: c->layers[l].bound |= SUB_WGATE; break;
    case P_WUP: c->layers[l].bound |= SUB_WUP; break;
    default: break;
  }
  return 0;
}

int ensure_activations(tgohip_ctx* c, int rows, int B) {
  const tgohip_model_cfg& m = c->cfg;
  const size_t d = m.hidden, qw = (size_t)m.heads * m.head_dim, kw = (size_t)m.kv_heads * m.head_dim;
  const size_t f = m.ffn;
  const size_t act_el = c->precision ? 4 : 2;
  int rc = 0;
  if (rows > c->rows_cap) {
    if ((rc = c->h.ensure(rows * d * 4))) return rc;
    if ((rc = c->xn.ensure(rows * d * 4))) return rc;
    if ((rc = c->qkv.ensure(rows * (qw + 2 * kw) * 4))) return rc;
    if ((rc = c->q.ensure(rows * qw * 4))) return rc;
    if ((rc = c->attn.ensure(rows * qw * 4))) return rc;
    if ((rc = c->act.ensure(rows * f * act_el + 256))) return rc;
    if ((rc = c->rows.ensure((size_t)rows * 8))) return rc;
    if ((rc = c->rope.ensure((size_t)rows * 32 * sizeof(float4_t)))) return rc;
    c->rows_cap = rows;
  }
  if (B > c->batch_cap) {
    if ((rc = c->lastn.ensure((size_t)B * d * 4))) return rc;
    if ((rc = c->logits.ensure((size_t)B * m.vocab * 4))) return rc;
    if ((rc = c->argmax.ensure((size_t)B * 4))) return rc;
    if ((rc = c->margin.ensure((size_t)B * 8))) return rc;
    if ((rc = c->amax_part.ensure(argmax_scratch_bytes(B, m.vocab)))) return rc;
    c->batch_cap = B;
  }
  // split-K workspace: the largest any projection of this step may ask for
  size_t ws = 0;
  for (const Layer& L : c->layers)
    for (const PackedWeight* w : {&L.qkv, &L.wo, &L.gateup, &L.down})
      if (w->form >= 0) ws = std::max(ws, gemm_workspace_bytes(*w, rows, c->ncu));
  if (c->lm_head.form >= 0) ws = std::max(ws, gemm_workspace_bytes(c->lm_head, B, c->ncu));
  if ((rc = c->gemm_ws.ensure(ws + 256))) return rc;
  return 0;
}

int ensure_attn_parts(tgohip_ctx* c, int parts) {
  int rc = c->part_o.ensure((size_t)std::max(parts, 1) * kAttnRowsP * 128 * 4);
  if (rc) return rc;
  return c->part_ml.ensure((size_t)std::max(parts, 1) * 2 * kAttnRowsP * 4);
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

const char* tgohip_last_error(void) { return g_err.c_str(); }
const char* tgohip_version(void) { return "tgohip 0.1 gfx950"; }

tgohip_ctx* tgohip_open(int device) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
    fail(TGOHIP_EDEVICE, "tgohip_open: no HIP device is visible");
    return nullptr;
  }
  if (device < 0 || device >= n) {
    fail(TGOHIP_EINVAL, "tgohip_open: device " + std::to_string(device) + " of " + std::to_string(n));
    return nullptr;
  }
  if (hipSetDevice(device) != hipSuccess) {
    fail(TGOHIP_EDEVICE, "tgohip_open: hipSetDevice failed");
    return nullptr;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
    fail(TGOHIP_EDEVICE, "tgohip_open: hipGetDeviceProperties failed");
    return nullptr;
  }
  if (std::string(prop.gcnArchName).find("gfx950") == std::string::npos) {
    fail(TGOHIP_EDEVICE, std::string("tgohip_open: this library is built for gfx950 and the device is ") +
                             prop.gcnArchName);
    return nullptr;
  }
  void* scr = nullptr;
  if (scratch_setup(device, &scr)) return nullptr;
  auto* c = new tgohip_ctx();
  c->device = device;
  c->ncu = prop.multiProcessorCount;
  c->scratch = scr;
  if (hipStreamCreate(&c->own_stream) != hipSuccess ||
      hipEventCreateWithFlags(&c->staged, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&c->ev0, hipEventDisableSystemFence) != hipSuccess ||
      hipEventCreate(&c->ev1) != hipSuccess) {
    fail(TGOHIP_EDEVICE, "tgohip_open: stream/event creation failed");
    delete c;
    return nullptr;
  }
  c->stream = c->own_stream;
  return c;
}

void tgohip_close(tgohip_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  for (void* p : c->allocs) (void)hipFree(p);
  c->allocs.clear();
  for (DevBuf* b : {&c->h, &c->xn, &c->qkv, &c->q, &c->attn, &c->act, &c->lastn, &c->logits,
                    &c->argmax, &c->margin, &c->amax_part, &c->meta, &c->gemm_ws, &c->part_o, &c->part_ml,
                    &c->rows, &c->rope})
    b->release();
  if (c->kc) (void)hipFree(c->kc);
  if (c->vc) (void)hipFree(c->vc);
  if (c->pinned) (void)hipHostFree(c->pinned);
  for (hipEvent_t e : c->prof_ev) (void)hipEventDestroy(e);
  (void)hipEventDestroy(c->staged);
  (void)hipEventDestroy(c->ev0);
  (void)hipEventDestroy(c->ev1);
  (void)hipStreamDestroy(c->own_stream);
  delete c;
}

void* tgohip_stream(tgohip_ctx* c) { return (void*)c->stream; }

// Launch on a caller's stream (for instance torch's current stream) instead
// of the context's own. NULL is the device's default stream.
int tgohip_set_stream(tgohip_ctx* c, void* stream) {
  TGOHIP_HIP(hipStreamSynchronize(c->stream));
  c->stream = (hipStream_t)stream;
  return 0;
}

int tgohip_use_own_stream(tgohip_ctx* c) {
  TGOHIP_HIP(hipStreamSynchronize(c->stream));
  c->stream = c->own_stream;
  return 0;
}

int tgohip_sync(tgohip_ctx* c) {
  TGOHIP_HIP(hipStreamSynchronize(c->stream));
  return 0;
}

int tgohip_set_cascade(tgohip_ctx* c, int min_sharers) {
  if (min_sharers != 0 && min_sharers < 2)
    return fail(TGOHIP_EINVAL, "cascade: min_sharers is 0 (off) or at least 2, not " +
                                   std::to_string(min_sharers));
  c->cascade = min_sharers;
  return 0;
}

int tgohip_set_precision(tgohip_ctx* c, int mode) {
  if (mode != 0 && mode != 1) return fail(TGOHIP_EINVAL, "precision is 0 (f16 activations) or 1 (f32 activations)");
  c->precision = mode;
  c->rows_cap = 0;  // activation dtype changed: regrow
  return 0;
}

int tgohip_config(tgohip_ctx* c, const tgohip_model_cfg* m) {
  if (c->configured) return fail(TGOHIP_ESTATE, "config: the context is already configured");
  if (m->layers <= 0 || m->hidden <= 0 || m->heads <= 0 || m->kv_heads <= 0 || m->vocab <= 0 ||
      m->ffn <= 0)
    return fail(TGOHIP_EINVAL, "config: every dimension is positive");
  if (m->head_dim != kHeadDim)
    return fail(TGOHIP_EINVAL, "config: head_dim is " + std::to_string(m->head_dim) +
                                   "; the kernels are built for 128 (every Qwen3 size)");
  if (m->heads % m->kv_heads != 0)
    return fail(TGOHIP_EINVAL, "config: num_attention_heads " + std::to_string(m->heads) +
                                   " is not a multiple of num_key_value_heads " +
                                   std::to_string(m->kv_heads));
  if (m->hidden % 64 != 0 || m->ffn % 64 != 0 || m->vocab % 32 != 0)
    return fail(TGOHIP_EINVAL, "config: hidden and ffn are multiples of 64 and vocab of 32");
  if (m->block <= 0) return fail(TGOHIP_EINVAL, "config: block is " + std::to_string(m->block));
  if (!(m->rms_eps > 0)) return fail(TGOHIP_EINVAL, "config: rms_norm_eps must be positive");
  c->cfg = *m;
  c->layers.assign(m->layers, Layer());
  // theta_i = base^(-2i/d_h) in double, once (internal/oracle/rope.go:119).
  std::vector<double> inv(kHeadDim / 2);
  for (int i = 0; i < kHeadDim / 2; i++)
    inv[i] = std::pow((double)m->rope_theta, -2.0 * (double)i / (double)kHeadDim);
  int rc = alloc_owned(c, (void**)&c->inv_freq, inv.size() * sizeof(double));
  if (rc) return rc;
  TGOHIP_HIP(hipMemcpy(c->inv_freq, inv.data(), inv.size() * sizeof(double), hipMemcpyHostToDevice));
  c->configured = true;
  return 0;
}

int tgohip_get_config(tgohip_ctx* c, tgohip_model_cfg* out) {
  if (!c->configured) return fail(TGOHIP_ESTATE, "config: the context is not configured");
  *out = c->cfg;
  return 0;
}

int tgohip_weight(tgohip_ctx* c, const char* port, int form, int K, int N, const void* plane,
                  const void* scales, const void* zeros) {
  if (!c->configured) return fail(TGOHIP_ESTATE, "weight: configure the context first");
  int l;
  const PortKind kind = parse_port(port, l);
  if (kind == P_BAD || (l >= 0 && l >= c->cfg.layers))
    return fail(TGOHIP_EINVAL, std::string("weight: no port named ") + port);
  if (kind == P_EMBED) {
    if (form != TGOHIP_FORM_F16 && form != TGOHIP_FORM_I8)
      return fail(TGOHIP_EINVAL, "weight embed: the embedding is gathered by row and is f16 or int8 "
                                 "(weights/weights.go:543-545 caps int4 to int8)");
    if (K != c->cfg.vocab || N != c->cfg.hidden)
      return fail(TGOHIP_EINVAL, "weight embed is [" + std::to_string(K) + "," + std::to_string(N) +
                                     "] and the config asks for [vocab, hidden]");
    free_owned(c, c->embed);
    free_owned(c, c->embed_scales);
    c->embed_scales = nullptr;
    int rc = alloc_owned(c, &c->embed, plane_bytes(form, K, N));
    if (rc) return rc;
    TGOHIP_HIP(hipMemcpy(c->embed, plane, plane_bytes(form, K, N), hipMemcpyHostToDevice));
    if (form == TGOHIP_FORM_I8) {
      rc = alloc_owned(c, (void**)&c->embed_scales, scale_count(form, K, N) * 2);
      if (rc) return rc;
      TGOHIP_HIP(hipMemcpy(c->embed_scales, scales, scale_count(form, K, N) * 2, hipMemcpyHostToDevice));
    }
    c->embed_form = form;
    return 0;
  }
  int rc = check_shape(form, K, N, port);
  if (rc) return rc;
  Canon cn;
  rc = canon_upload(c, cn, form, K, N, plane, scales, zeros);
  if (rc) return rc;
  rc = place_weight(c, kind, l, form, K, N, cn, port);
  if (rc) return rc;
  TGOHIP_HIP(hipStreamSynchronize(c->stream));
  return 0;
}

// An f32 plane quantized on the device: the canonical codes of
// tgohip_quantize_int8 / tgohip_quantize_int4 (bit for bit), then placed as
// tgohip_weight places them.
int tgohip_weight_f32(tgohip_ctx* c, const char* port, int form, int K, int N, const float* w) {
  if (!c->configured) return fail(TGOHIP_ESTATE, "weight: configure the context first");
  int l;
  const PortKind kind = parse_port(port, l);
  if (kind == P_BAD || (l >= 0 && l >= c->cfg.layers))
    return fail(TGOHIP_EINVAL, std::string("weight: no port named ") + port);
  if (kind == P_EMBED) {
    if (form != TGOHIP_FORM_I8)
      return fail(TGOHIP_EINVAL, "weight_f32 embed: the device quantizes the gathered embedding to "
                                 "int8 (weights/weights.go:543-545 caps int4 to int8; f16 converts "
                                 "on the host)");
    if (K != c->cfg.vocab || N != c->cfg.hidden)
      return fail(TGOHIP_EINVAL, "weight embed is [" + std::to_string(K) + "," + std::to_string(N) +
                                     "] and the config asks for [vocab, hidden]");
    if (!w) return fail(TGOHIP_EINVAL, "weight: the plane is missing");
    const size_t n = (size_t)K * N;
    float* dw = nullptr;
    TGOHIP_HIP(hipMalloc((void**)&dw, n * sizeof(float)));
    DevFree hold{dw};
    TGOHIP_HIP(hipMemcpyAsync(dw, w, n * sizeof(float), hipMemcpyHostToDevice, c->stream));
    free_owned(c, c->embed);
    free_owned(c, c->embed_scales);
    c->embed_scales = nullptr;
    int rc = alloc_owned(c, &c->embed, plane_bytes(form, K, N));
    if (rc) return rc;
    rc = alloc_owned(c, (void**)&c->embed_scales, scale_count(form, K, N) * 2);
    if (rc) return rc;
    launch_quantize_i8(dw, n, (int8_t*)c->embed, (uint16_t*)c->embed_scales, c->stream);
    TGOHIP_HIP(hipGetLastError());
    TGOHIP_HIP(hipStreamSynchronize(c->stream));
    c->embed_form = form;
    return 0;
  }
  int rc = check_shape(form, K, N, port);
  if (rc) return rc;
  Canon cn;
  if ((rc = canon_quantize(c, cn, form, K, N, w))) return rc;
  if ((rc = place_weight(c, kind, l, form, K, N, cn, port))) return rc;
  TGOHIP_HIP(hipStreamSynchronize(c->stream));
  return 0;
}

int tgohip_gain(tgohip_ctx* c, const char* port, const float* g, int width) {
  if (!c->configured) return fail(TGOHIP_ESTATE, "gain: configure the context first");
  float** dst = nullptr;
  int want = 0;
  if (!strcmp(port, "final_norm")) {
    dst = &c->g_final;
    want = c->cfg.hidden;
  } else {
    char* end = nullptr;
    const long l = strtol(port, &end, 10);
    if (end == port || *end != '.' || l < 0 || l >= c->cfg.layers)
      return fail(TGOHIP_EINVAL, std::string("gain: no port named ") + port);
    const char* name = end + 1;
    Layer& L = c->layers[l];
    if (!strcmp(name, "attn_norm")) { dst = &L.g_attn; want = c->cfg.hidden; }
    else if (!strcmp(name, "ffn_norm")) { dst = &L.g_ffn; want = c->cfg.hidden; }
    else if (!strcmp(name, "qnorm")) { dst = &L.g_q; want = kHeadDim; }
    else if (!strcmp(name, "knorm")) { dst = &L.g_k; want = kHeadDim; }
    else return fail(TGOHIP_EINVAL, std::string("gain: no port named ") + port);
  }
  if (width != want)
    return fail(TGOHIP_EINVAL, std::string("gain ") + port + " is " + std::to_string(width) +
                                   " wide and the config asks for " + std::to_string(want));
  if (!*dst) {
    int rc = alloc_owned(c, (void**)dst, (size_t)want * 4);
    if (rc) return rc;
  }
  TGOHIP_HIP(hipMemcpy(*dst, g, (size_t)want * 4, hipMemcpyHostToDevice));
  return 0;
}

int tgohip_synth_weights(tgohip_ctx* c, uint64_t seed, int form, double sigma) {
  if (!c->configured) return fail(TGOHIP_ESTATE, "synth: configure the context first");
  const tgohip_model_cfg& m = c->cfg;
  const int d = m.hidden, qw = m.heads * m.head_dim, kw = m.kv_heads * m.head_dim, f = m.ffn;
  int rc;
  // embedding: F16 under F16, else int8 (stream 1)
  {
    const int ef = form == TGOHIP_FORM_F16 ? TGOHIP_FORM_F16 : TGOHIP_FORM_I8;
    free_owned(c, c->embed);
    free_owned(c, c->embed_scales);
    c->embed_scales = nullptr;
    if ((rc = alloc_owned(c, &c->embed, plane_bytes(ef, m.vocab, d)))) return rc;
    const size_t n = (size_t)m.vocab * d;
    if (ef == TGOHIP_FORM_F16) {
      launch_synth_f16(seed, 1 * 4, n, sigma, (uint16_t*)c->embed, c->stream);
    } else {
      if ((rc = alloc_owned(c, (void**)&c->embed_scales, scale_count(ef, m.vocab, d) * 2))) return rc;
      launch_synth_i8(seed, 1 * 4, n, (int8_t*)c->embed, c->stream);
      launch_synth_absf16(seed, 1 * 4 + 1, scale_count(ef, m.vocab, d), sigma / 64.0, c->embed_scales, c->stream);
    }
    c->embed_form = ef;
  }
  {
    Canon cn;
    if ((rc = check_shape(form, d, m.vocab, "lm_head"))) return rc;
    if ((rc = canon_synth(c, cn, seed, 3, form, d, m.vocab, sigma))) return rc;
    if ((rc = place_weight(c, P_LMHEAD, -1, form, d, m.vocab, cn, "lm_head"))) return rc;
    TGOHIP_HIP(hipStreamSynchronize(c->stream));
  }
  // Gains: multiples of 1/8 in [-2, 2) from (seed, port stream), the CPU
  // restatement's orc_synth_gain (final_norm is stream 2, a layer's gains
  // streams (l+1)*64 + 0, 5, 6, 7).
  auto gain = [&](float** dst, int w, uint64_t stream) -> int {
    if (!*dst) {
      int r = alloc_owned(c, (void**)dst, (size_t)w * 4);
      if (r) return r;
    }
    launch_synth_gain(seed, stream * 4, (size_t)w, *dst, c->stream);
    return 0;
  };
  if ((rc = gain(&c->g_final, d, 2))) return rc;
  struct P { PortKind k; int p; int K, N; const char* name; };
  const P ports[] = {{P_WQ, 1, d, qw, "wq"}, {P_WK, 2, d, kw, "wk"}, {P_WV, 3, d, kw, "wv"},
                     {P_WO, 4, qw, d, "wo"}, {P_WGATE, 8, d, f, "wgate"}, {P_WUP, 9, d, f, "wup"},
                     {P_WDOWN, 10, f, d, "wdown"}};
  for (int l = 0; l < m.layers; l++) {
    Layer& L = c->layers[l];
    const uint64_t ls = (uint64_t)(l + 1) * 64;
    if ((rc = gain(&L.g_attn, d, ls + 0)) || (rc = gain(&L.g_ffn, d, ls + 7)) ||
        (rc = gain(&L.g_q, kHeadDim, ls + 5)) || (rc = gain(&L.g_k, kHeadDim, ls + 6)))
      return rc;
    for (const P& p : ports) {
      Canon cn;
      const std::string name = std::to_string(l) + "." + p.name;
      if ((rc = check_shape(form, p.K, p.N, name.c_str()))) return rc;
      if ((rc = canon_synth(c, cn, seed, (uint64_t)(l + 1) * 64 + p.p, form, p.K, p.N, sigma))) return rc;
      if ((rc = place_weight(c, p.k, l, form, p.K, p.N, cn, name.c_str()))) return rc;
      TGOHIP_HIP(hipStreamSynchronize(c->stream));
    }
  }
  return 0;
}

int tgohip_kv_alloc(tgohip_ctx* c, int positions) {
  if (!c->configured) return fail(TGOHIP_ESTATE, "kv_alloc: configure the context first");
  if ((int64_t)positions * c->cfg.kv_heads * kHeadDim >= (int64_t)1 << 31)
    return fail(TGOHIP_EINVAL, "kv_alloc: one layer of the pool is addressed with 32-bit element "
                               "offsets; " + std::to_string(positions) + " positions exceed it");
  const int blocks = positions / c->cfg.block;
  if (blocks < 1)
    return fail(TGOHIP_EINVAL, "kv_alloc: a shared cache of " + std::to_string(positions) +
                                   " positions holds no whole block of " + std::to_string(c->cfg.block) +
                                   "; it needs at least one");
  const int pos = blocks * c->cfg.block;
  const size_t n = (size_t)c->cfg.layers * pos * c->cfg.kv_heads * kHeadDim;
  if (c->kc) (void)hipFree(c->kc);
  if (c->vc) (void)hipFree(c->vc);
  c->kc = c->vc = nullptr;
  hipError_t e = hipMalloc((void**)&c->kc, n * 2);
  if (e == hipSuccess) e = hipMalloc((void**)&c->vc, n * 2);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    if (c->kc) (void)hipFree(c->kc);
    c->kc = c->vc = nullptr;  // no half pool: a step then refuses for want of one
    c->kv_positions = 0;
    return fail(TGOHIP_ENOMEM, "kv_alloc: the shared prefix cache needs " + std::to_string(n * 2) +
                                   " bytes per state at " + std::to_string(pos) +
                                   " positions and the device refused it");
  }
  // Zeroed (blocks.go:117-137).
  TGOHIP_HIP(hipMemsetAsync(c->kc, 0, n * 2, c->stream));
  TGOHIP_HIP(hipMemsetAsync(c->vc, 0, n * 2, c->stream));
  TGOHIP_HIP(hipStreamSynchronize(c->stream));
  c->kv_positions = pos;
  return 0;
}

int tgohip_kv_pointers(tgohip_ctx* c, void** k, void** v, int* positions) {
  *k = c->kc;
  *v = c->vc;
  *positions = c->kv_positions;
  return 0;
}

// ---- the batched step ------------------------------------------------------
}  // extern "C"

namespace {

// One step's device work, enqueued on c->stream without waiting: the ports
// staged and uploaded, every kernel launched, ev_begin / ev_end recorded
// around them. The argmax of every member is left in c->argmax.
// Algorithmic bytes and flops of one launch of each profiled kernel kind.
struct ProfStep {
  double bytes[TGOHIP_PROF_KINDS] = {};
  double flops[TGOHIP_PROF_KINDS] = {};
};

struct StepLaunch {
  const int32_t* feed = nullptr;  // ids with bit 31 set take feed[member] (device)
  int keep_idle = 0;              // argmax leaves the entries of idle members as they are
  hipEvent_t ev_begin = nullptr, ev_end = nullptr;
  int prof_set = 0;               // which set of profile events
  ProfStep prof;                  // out: per-launch algorithmic bytes and flops
};

// A projection's algorithmic bytes (weights once, activations in, output out;
// a residual add reads and writes h) and flops, 2*M*K*N. xk: XK_F16 (2 bytes
// per activation), XK_F32 or XK_X2 (4).
void gemm_algorithmic(const PackedWeight& w, int M, int xk, int epi, double& bytes, double& flops) {
  const double halves = (double)packed_scale_halves(w.form, w.K, w.N);
  bytes = (double)packed_payload_bytes(w.form, w.K, w.N) +
          halves * 2 * (w.form == TGOHIP_FORM_I4_TGO ? 2 : 1) +
          (double)M * w.K * (xk == XK_F16 ? 2 : 4);
  switch (epi) {
    case EPI_RESID: bytes += (double)M * w.N * 8; break;
    case EPI_SWIGLU_F16: bytes += (double)M * w.N / 2 * 2; break;
    case EPI_SWIGLU_F32:
    case EPI_SWIGLU_X2: bytes += (double)M * w.N / 2 * 4; break;
    case EPI_F16: bytes += (double)M * w.N * 2; break;
    default: bytes += (double)M * w.N * 4; break;
  }
  flops = 2.0 * M * w.K * w.N;
}

int step_launch(tgohip_ctx* c, const tgohip_batch_step* s, StepLaunch& o) {
  if (!c->configured) return fail(TGOHIP_ESTATE, "step: configure the context first");
  if (!c->kc) return fail(TGOHIP_ESTATE, "step: a batched step needs a shared block pool (kv_alloc)");
  const tgohip_model_cfg& m = c->cfg;
  if (c->embed_form < 0 || c->lm_head.form < 0 || !c->g_final)
    return fail(TGOHIP_ESTATE, "step: the embedding, lm_head and final_norm are bound first");
  for (int l = 0; l < m.layers; l++) {
    const Layer& L = c->layers[l];
    static const std::pair<int, const char*> subs[] = {
        {SUB_WQ, "wq"}, {SUB_WK, "wk"}, {SUB_WV, "wv"}, {SUB_WGATE, "wgate"}, {SUB_WUP, "wup"}};
    for (const auto& sp : subs)
      if (!(L.bound & sp.first))
        return fail(TGOHIP_ESTATE, "step: layer " + std::to_string(l) + " has an unbound port (" +
                                       std::to_string(l) + "." + sp.second + ")");
    if (L.wo.form < 0 || L.down.form < 0 || !L.g_attn || !L.g_ffn || !L.g_q || !L.g_k)
      return fail(TGOHIP_ESTATE, "step: layer " + std::to_string(l) + " has an unbound port");
  }
  const int T = s->rows, B = s->batch;
  if (T <= 0 || B <= 0) return fail(TGOHIP_EINVAL, "step: rows and batch are positive");
  for (int t = 0; t < T; t++) {
    if (o.feed && (s->ids[t] >> 31)) {
      if ((s->ids[t] & 0x7fffffffu) >= (uint32_t)B)
        return fail(TGOHIP_EINVAL, "step: row " + std::to_string(t) + " takes the token of member " +
                                       std::to_string(s->ids[t] & 0x7fffffffu) + " of " +
                                       std::to_string(B));
      continue;
    }
    if (s->ids[t] >= (uint32_t)m.vocab)
      return fail(TGOHIP_EINVAL, "step: row " + std::to_string(t) + " token id " +
                                     std::to_string(s->ids[t]) + " is outside the vocabulary");
  }
  const bool derived = !s->posq;
  if (derived != !s->posk || derived != !s->slots)
    return fail(TGOHIP_EINVAL, "step: posq, posk and slots are given together, or all three are "
                               "null and derived on the device from lengths, extents and pages");
  for (int b = 0; b < B; b++) {
    if (s->extents[b] > 0 && s->last[b] >= (uint32_t)T)
      return fail(TGOHIP_EINVAL, "step: member " + std::to_string(b) + " reads logits from row " +
                                     std::to_string(s->last[b]) + " of " + std::to_string(T));
  }
  AttnPlan plan;
  int rc = attn_build_plan(T, B, s->lengths, s->extents, s->pages, s->max_pages, m.block,
                           c->kv_positions, m.heads, m.kv_heads, plan, c->cascade,
                           c->precision == 1);
  if (rc) return rc;
  int pad = -1;
  for (int b = 0; b < B; b++)
    if (s->extents[b] > 0) pad = b;
  if (derived && pad < 0)
    return fail(TGOHIP_EINVAL, "step: every member contributes nothing; there are no positions "
                               "to derive");
  // Rows past the members' (sum of extents) are a bucket's padding
  // (batch.go:362-366, model/batch.go:140-150): attention leaves them inert,
  // no member reads their logits, and a slot at or past capacity drops their
  // K/V write (plan.go:180-192). Such rows change nothing, so the step runs
  // over the members' rows only: a 1152-row step bucketed to 2048 costs what
  // the 1152 rows cost. A padding row whose slot is in the pool (ports not
  // packed by NewBatchStep) would write K/V, and a member reading its logits
  // from a padding row needs it computed: then every row runs.
  int Tw = T;
  if (plan.claimed > 0 && plan.claimed < T) {
    bool inert = true;
    if (!derived)
      for (int t = plan.claimed; t < T && inert; t++) inert = s->slots[t] >= (uint32_t)c->kv_positions;
    for (int b = 0; b < B && inert; b++)
      if (s->extents[b] > 0 && s->last[b] >= (uint32_t)plan.claimed) inert = false;
    if (inert) Tw = plan.claimed;
  }
  // The head's rows: only members that worked need logits (an idle member's
  // row is zero and its token -1), so the final norm, the LM head and the
  // greedy selection run over those, compacted: at C4 128-130 of 136 slots,
  // and the LM head's 64-row tiles 2 instead of 3.
  std::vector<uint32_t> head_last;
  std::vector<int32_t> head_idx(B, -1);
  c->head_rows.clear();
  for (int b = 0; b < B; b++)
    if (s->extents[b] > 0) {
      head_idx[b] = (int32_t)c->head_rows.size();
      c->head_rows.push_back(b);
      head_last.push_back(s->last[b]);
    }
  const int nh = (int)c->head_rows.size();
  const bool compact = nh > 0 && nh < B;
  if (!compact) c->head_rows.clear();
  const int HB = compact ? nh : B;  // rows of the head
  if ((rc = ensure_activations(c, Tw, B))) return rc;
  if ((rc = ensure_attn_parts(c, plan.parts))) return rc;

  // One staged upload of every port (batch.go:385-405).
  Stager sg;
  const size_t o_ids = sg.add(s->ids, (size_t)Tw * 4);
  const size_t o_posq = derived ? 0 : sg.add(s->posq, (size_t)Tw * m.heads * 4);
  const size_t o_posk = derived ? 0 : sg.add(s->posk, (size_t)Tw * m.kv_heads * 4);
  const size_t o_slots = derived ? 0 : sg.add(s->slots, (size_t)Tw * 4);
  const size_t o_len = sg.add(s->lengths, (size_t)B * 4);
  const size_t o_ext = sg.add(s->extents, (size_t)B * 4);
  const size_t o_last = sg.add(s->last, (size_t)B * 4);
  const size_t o_pages = sg.add(s->pages, (size_t)B * s->max_pages * 4);
  const size_t o_cu = sg.add(plan.cu.data(), (size_t)B * 4);
  const size_t o_items = sg.add(plan.items.data(), plan.items.size() * sizeof(AttnItem));
  const size_t o_comb = sg.add(plan.combines.data(), plan.combines.size() * sizeof(AttnCombine));
  const size_t o_seql = sg.add(plan.seqlist.data(), plan.seqlist.size() * sizeof(int32_t));
  const size_t o_hlast = compact ? sg.add(head_last.data(), (size_t)nh * 4) : 0;
  const size_t o_hidx = compact ? sg.add(head_idx.data(), (size_t)B * 4) : 0;
  if ((rc = sg.upload(c))) return rc;
  const hipStream_t st = c->stream;
  TGOHIP_HIP(hipEventRecord(o.ev_begin, st));

  const uint32_t* d_ids = sg.dev<uint32_t>(c, o_ids);
  const uint32_t* d_ext = sg.dev<uint32_t>(c, o_ext);
  AttnDevPlan dp{sg.dev<AttnItem>(c, o_items), sg.dev<AttnCombine>(c, o_comb),
                 sg.dev<int32_t>(c, o_seql), sg.dev<int32_t>(c, o_cu),
                 sg.dev<uint32_t>(c, o_len), d_ext, sg.dev<uint32_t>(c, o_pages),
                 (float*)c->part_o.p, (float*)c->part_ml.p};
  // Precision mode 1 (tgo's f32 arithmetic): each projection's input is an
  // activation pair written by its producer (rmsnorm, attention, the SwiGLU
  // epilogue) and q is f32; mode 0: f16 activations and q.
  const bool f32act = c->precision == 1;
  const int xk = f32act ? XK_X2 : XK_F16;
  const int outf = f32act ? OUT_X2 : OUT_F16;
  const int qf16 = f32act ? 0 : 1;
  const int swiglu = f32act ? EPI_SWIGLU_X2 : EPI_SWIGLU_F16;
  const float scale = (float)(1.0 / std::sqrt((double)m.head_dim));  // session.go:821-823
  float* h = (float*)c->h.p;
  const size_t layer_kv = (size_t)c->kv_positions * m.kv_heads * kHeadDim;
  float* ws = (float*)c->gemm_ws.p;
  const size_t wsb = c->gemm_ws.bytes;

  // Algorithmic bytes of one attention launch: every cached position a
  // claimed row reads, once (K and V, all kv heads), plus q read and out written;
  // flops 4 * d_h * H per visible (query, key) pair.
  o.prof = ProfStep();
  hipEvent_t* pev = nullptr;
  constexpr int NK = TGOHIP_PROF_KINDS;
  if (c->profile) {
    double& ab = o.prof.bytes[TGOHIP_PROF_ATTN];
    double pairs = 0;
    for (int b = 0; b < B; b++) {
      const double L = s->lengths[b], n = s->extents[b];
      if (n > 0) ab += L * m.kv_heads * kHeadDim * 2 * 2;
      pairs += n * (L - n) + n * (n + 1) / 2;
    }
    ab += (double)plan.claimed * m.heads * kHeadDim * (f32act ? 4 + 4 : 2 + 2);  // q in, out
    ab -= (double)plan.shared_positions * m.kv_heads * kHeadDim * 2 * 2;  // read once
    o.prof.flops[TGOHIP_PROF_ATTN] = 4.0 * kHeadDim * m.heads * pairs;
    const Layer& L0 = c->layers[0];
    gemm_algorithmic(L0.qkv, Tw, xk, EPI_F32, o.prof.bytes[TGOHIP_PROF_QKV], o.prof.flops[TGOHIP_PROF_QKV]);
    gemm_algorithmic(L0.wo, Tw, xk, EPI_RESID, o.prof.bytes[TGOHIP_PROF_O], o.prof.flops[TGOHIP_PROF_O]);
    gemm_algorithmic(L0.gateup, Tw, xk, swiglu, o.prof.bytes[TGOHIP_PROF_GATEUP],
                     o.prof.flops[TGOHIP_PROF_GATEUP]);
    gemm_algorithmic(L0.down, Tw, xk, EPI_RESID, o.prof.bytes[TGOHIP_PROF_DOWN], o.prof.flops[TGOHIP_PROF_DOWN]);
    gemm_algorithmic(c->lm_head, HB, xk, EPI_F32, o.prof.bytes[TGOHIP_PROF_LMHEAD],
                     o.prof.flops[TGOHIP_PROF_LMHEAD]);
    while (c->prof_ev.size() < (size_t)2 * m.layers * NK * 2) {
      // timing only: no system-scope fence (an L2 write-back each, which
      // left a ~6 us gap on both sides of every attention launch)
      hipEvent_t e;
      TGOHIP_HIP(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
      c->prof_ev.push_back(e);
    }
    pev = c->prof_ev.data() + (size_t)o.prof_set * m.layers * NK * 2;
  }
  // events around kernel `kind` of layer l, when profiled
  auto mark = [&](int kind, int l, int end) -> int {
    if (pev && (c->prof_mask >> kind & 1) && (kind == TGOHIP_PROF_LMHEAD || l % c->prof_stride == 0))
      TGOHIP_HIP(hipEventRecord(pev[((size_t)l * NK + kind) * 2 + end], st));
    return 0;
  };
  launch_embed(d_ids, Tw, c->embed, c->embed_scales, c->embed_form, m.hidden, h, st, o.feed);
  uint32_t* d_rowpos = (uint32_t*)c->rows.p;
  uint32_t* d_rowslot = d_rowpos + Tw;
  if (derived) {
    launch_derive_rows(DeriveArgs{dp.cu, dp.lengths, d_ext, dp.pages, B, s->max_pages, m.block,
                                  plan.claimed, pad, Tw, c->kv_positions, d_rowpos, d_rowslot},
                       st);
    launch_rope_table(d_rowpos, Tw, c->inv_freq, (float4_t*)c->rope.p, st);
  }
  // A split-K projection's partial planes are summed by the kernel that reads
  // its output next (in split order, so the result is the reduction's):
  // QKV's by qk_rope_kv, O's and down's (residual adds) by the following
  // rmsnorm. `pend` counts the planes of a residual add still owed to h.
  const size_t plane = split_plane_stride(Tw, m.hidden);
  int pend = 0;
  // tgo's arithmetic with device-derived rows: the QKV projection runs its
  // q/k-norm, RoPE and K/V write in its epilogue where its launch allows
  // (unsplit; at the C4 step's 1152 rows, not at 128); TGOHIP_FUSE_QK=0 keeps
  // the separate kernel. Both compute the same values.
  static const bool fuse_env = [] {
    const char* e = getenv("TGOHIP_FUSE_QK");
    return !(e && atoi(e) == 0);
  }();
  const bool fuse_ok = fuse_env && f32act && derived;
  for (int l = 0; l < m.layers; l++) {
    const Layer& L = c->layers[l];
    // per layer: a checkpoint's layers may hold different weight forms
    const bool fuse_qk = fuse_ok && gemm_qkrope_fusable(L.qkv, Tw, c->ncu);
    launch_rmsnorm(h, nullptr, Tw, L.g_attn, m.hidden, m.rms_eps, c->xn.p, outf, st, ws, pend, plane);
    int qkv_split = 0;
    QKRopeArgs qa{nullptr, 0, split_plane_stride(Tw, (m.heads + 2 * m.kv_heads) * kHeadDim),
                  L.g_q, L.g_k,
                  derived ? nullptr : sg.dev<uint32_t>(c, o_posq),
                  derived ? nullptr : sg.dev<uint32_t>(c, o_posk),
                  derived ? d_rowslot : sg.dev<uint32_t>(c, o_slots), derived ? d_rowpos : nullptr,
                  c->inv_freq, c->q.p, c->kc + l * layer_kv,
                  c->vc + l * layer_kv, m.heads, m.kv_heads, c->kv_positions, m.rms_eps, qf16,
                  derived ? (const float4_t*)c->rope.p : nullptr};
    if ((rc = mark(TGOHIP_PROF_QKV, l, 0))) return rc;
    if (fuse_qk) {
      // q/k-norm, RoPE and the K/V write in the projection's epilogue
      if ((rc = gemm_enqueue_qkrope(L.qkv, c->xn.p, Tw, qa, c->ncu, st))) return rc;
      if ((rc = mark(TGOHIP_PROF_QKV, l, 1))) return rc;
    } else {
      if ((rc = gemm_enqueue(L.qkv, c->xn.p, xk, Tw, c->qkv.p, EPI_F32, ws, wsb, c->ncu, st,
                             &qkv_split)))
        return rc;
      if ((rc = mark(TGOHIP_PROF_QKV, l, 1))) return rc;
      qa.qkv = qkv_split ? ws : (const float*)c->qkv.p;
      qa.nsplit = qkv_split;
      launch_qk_rope_kv(qa, Tw, st);
    }
    if ((rc = mark(TGOHIP_PROF_ATTN, l, 0))) return rc;
    if ((rc = attn_enqueue(plan, dp, c->q.p, qf16, c->kc + l * layer_kv, c->vc + l * layer_kv, c->attn.p,
                           outf, Tw, m.heads, m.kv_heads, s->max_pages, m.block, scale, st)))
      return rc;
    if ((rc = mark(TGOHIP_PROF_ATTN, l, 1))) return rc;
    if ((rc = mark(TGOHIP_PROF_O, l, 0))) return rc;
    if ((rc = gemm_enqueue(L.wo, c->attn.p, xk, Tw, h, EPI_RESID, ws, wsb, c->ncu, st, &pend)))
      return rc;
    if ((rc = mark(TGOHIP_PROF_O, l, 1))) return rc;
    launch_rmsnorm(h, nullptr, Tw, L.g_ffn, m.hidden, m.rms_eps, c->xn.p, outf, st, ws, pend, plane);
    if ((rc = mark(TGOHIP_PROF_GATEUP, l, 0))) return rc;
    if ((rc = gemm_enqueue(L.gateup, c->xn.p, xk, Tw, c->act.p, swiglu, ws, wsb, c->ncu, st)))
      return rc;
    if ((rc = mark(TGOHIP_PROF_GATEUP, l, 1))) return rc;
    if ((rc = mark(TGOHIP_PROF_DOWN, l, 0))) return rc;
    if ((rc = gemm_enqueue(L.down, c->act.p, xk, Tw, h, EPI_RESID, ws, wsb, c->ncu, st, &pend)))
      return rc;
    if ((rc = mark(TGOHIP_PROF_DOWN, l, 1))) return rc;
  }
  // The last layer's split residual add is summed for the Last rows only (the
  // head reads nothing else); h keeps the rows without it.
  launch_rmsnorm(h, sg.dev<uint32_t>(c, compact ? o_hlast : o_last), HB, c->g_final, m.hidden,
                 m.rms_eps, c->lastn.p, outf, st, ws, pend, plane);
  if ((rc = mark(TGOHIP_PROF_LMHEAD, 0, 0))) return rc;
  if ((rc = gemm_enqueue(c->lm_head, c->lastn.p, xk, HB, c->logits.p, EPI_F32, ws, wsb, c->ncu, st)))
    return rc;
  if ((rc = mark(TGOHIP_PROF_LMHEAD, 0, 1))) return rc;
  launch_argmax((float*)c->logits.p, B, m.vocab, d_ext, (int32_t*)c->argmax.p, c->amax_part.p, st,
                o.keep_idle, (double*)c->margin.p, 1, HB,
                compact ? sg.dev<int32_t>(c, o_hidx) : nullptr);
  TGOHIP_HIP(hipEventRecord(o.ev_end, st));
  TGOHIP_HIP(hipGetLastError());
  c->last_batch = B;
  return 0;
}

// Adds one landed step's profiled launches to the totals.
int profile_collect(tgohip_ctx* c, int prof_set, const ProfStep& ps) {
  constexpr int NK = TGOHIP_PROF_KINDS;
  const int L = c->cfg.layers;
  if (!c->profile || c->prof_ev.size() < (size_t)2 * L * NK * 2) return 0;
  const hipEvent_t* pev = c->prof_ev.data() + (size_t)prof_set * L * NK * 2;
  for (int k = 0; k < NK; k++) {
    if (!(c->prof_mask >> k & 1)) continue;
    const int stride = k == TGOHIP_PROF_LMHEAD ? L : c->prof_stride;
    for (int l = 0; l < L; l += stride) {
      float ms = 0;
      TGOHIP_HIP(hipEventElapsedTime(&ms, pev[((size_t)l * NK + k) * 2], pev[((size_t)l * NK + k) * 2 + 1]));
      c->prof_ms[k] += ms;
      c->prof_launches[k]++;
      c->prof_bytes[k] += ps.bytes[k];
      c->prof_flops[k] += ps.flops[k];
    }
  }
  return 0;
}

}  // namespace

extern "C" {

int tgohip_step(tgohip_ctx* c, const tgohip_batch_step* s, float* logits_out, int32_t* argmax_out,
                tgohip_timings* tm) {
  using clk = std::chrono::steady_clock;
  const auto t_start = clk::now();
  StepLaunch o;
  o.ev_begin = c->ev0;
  o.ev_end = c->ev1;
  int rc = step_launch(c, s, o);
  if (rc) return rc;
  const auto t_sub = clk::now();
  TGOHIP_HIP(hipEventSynchronize(c->ev1));
  const auto t_dev = clk::now();
  const tgohip_model_cfg& m = c->cfg;
  if (logits_out && c->head_rows.empty()) {
    TGOHIP_HIP(hipMemcpy(logits_out, c->logits.p, (size_t)s->batch * m.vocab * 4, hipMemcpyDeviceToHost));
  } else if (logits_out) {
    // compacted head rows: each member that worked gets its row, idle members zeros
    const size_t V = (size_t)m.vocab;
    std::vector<float> rows(c->head_rows.size() * V);
    TGOHIP_HIP(hipMemcpy(rows.data(), c->logits.p, rows.size() * 4, hipMemcpyDeviceToHost));
    memset(logits_out, 0, (size_t)s->batch * V * 4);
    for (size_t i = 0; i < c->head_rows.size(); i++)
      memcpy(logits_out + (size_t)c->head_rows[i] * V, rows.data() + i * V, V * 4);
  }
  if (argmax_out) TGOHIP_HIP(hipMemcpy(argmax_out, c->argmax.p, (size_t)s->batch * 4, hipMemcpyDeviceToHost));
  const auto t_end = clk::now();
  if ((rc = profile_collect(c, 0, o.prof))) return rc;
  if (tm) {
    float dev_ms = 0;
    (void)hipEventElapsedTime(&dev_ms, c->ev0, c->ev1);
    tm->submit_ms = std::chrono::duration<double, std::milli>(t_sub - t_start).count();
    tm->device_ms = dev_ms;
    tm->readback_ms = std::chrono::duration<double, std::milli>(t_end - t_dev).count();
  }
  return 0;
}

// The top-two margins of the last step's members (TopTwoMargin,
// internal/conformance/measure.go:91), waiting for the step to land.
int tgohip_step_margins(tgohip_ctx* c, double* out, int B) {
  if (B <= 0 || B > c->last_batch || !c->margin.p)
    return fail(TGOHIP_EINVAL, "step margins: " + std::to_string(B) + " members asked and the last "
                               "step held " + std::to_string(c->last_batch));
  TGOHIP_HIP(hipStreamSynchronize(c->stream));
  TGOHIP_HIP(hipMemcpy(out, c->margin.p, (size_t)B * 8, hipMemcpyDeviceToHost));
  return 0;
}

// ---- op level ---------------------------------------------------------------
// Greedy selection over B rows of V logits in device memory
// (sample/stages.go:196-206 argmax; TopTwoMargin of
// internal/conformance/measure.go:91 when margins is not null).
int tgohip_greedy(tgohip_ctx* c, const float* logits, int B, int V, int32_t* ids, double* margins) {
  if (B < 0) return fail(TGOHIP_EINVAL, "greedy: " + std::to_string(B) + " rows");
  if (V < 2)
    return fail(TGOHIP_EINVAL, "greedy: a vocabulary of " + std::to_string(V) +
                                   " logits; the top-two margin is over at least two");
  if (B == 0) return 0;
  if (!logits || !ids) return fail(TGOHIP_EINVAL, "greedy: logits and ids are device buffers");
  int rc;
  if ((rc = c->amax_part.ensure(argmax_scratch_bytes(B, V)))) return rc;
  // the logits are only read (no idle rows to zero)
  launch_argmax(const_cast<float*>(logits), B, V, nullptr, ids, c->amax_part.p, c->stream, 0,
                margins, 0);
  TGOHIP_HIP(hipGetLastError());
  return 0;
}

int tgohip_paged_attention(tgohip_ctx* c, const void* q, int q_dtype, int T, int H, int H_kv,
                           int head_dim, const void* k, const void* v, int capacity, int B,
                           const uint32_t* lengths, const uint32_t* extents, const uint32_t* pages,
                           int max_pages, int block, float scale, void* out, int out_dtype) {
  if (head_dim != kHeadDim)
    return fail(TGOHIP_EINVAL, "attention: head_dim is " + std::to_string(head_dim) +
                                   "; the kernel is built for 128");
  if (T < 0 || B < 0 || capacity <= 0) return fail(TGOHIP_EINVAL, "attention: T, B and capacity");
  if ((int64_t)capacity * H_kv * kHeadDim >= (int64_t)1 << 31)
    return fail(TGOHIP_EINVAL, "attention: the cache view exceeds 32-bit element offsets");
  AttnPlan plan;
  int rc = attn_build_plan(T, B, lengths, extents, pages, max_pages, block, capacity, H, H_kv, plan,
                           c->cascade, q_dtype != TGOHIP_F16);
  if (rc) return rc;
  if ((rc = ensure_attn_parts(c, plan.parts))) return rc;
  Stager sg;
  const size_t o_len = sg.add(lengths, (size_t)B * 4);
  const size_t o_ext = sg.add(extents, (size_t)B * 4);
  const size_t o_pages = sg.add(pages, (size_t)B * max_pages * 4);
  const size_t o_cu = sg.add(plan.cu.data(), (size_t)B * 4);
  const size_t o_items = sg.add(plan.items.data(), plan.items.size() * sizeof(AttnItem));
  const size_t o_comb = sg.add(plan.combines.data(), plan.combines.size() * sizeof(AttnCombine));
  const size_t o_seql = sg.add(plan.seqlist.data(), plan.seqlist.size() * sizeof(int32_t));
  if ((rc = sg.upload(c))) return rc;
  AttnDevPlan dp{sg.dev<AttnItem>(c, o_items), sg.dev<AttnCombine>(c, o_comb),
                 sg.dev<int32_t>(c, o_seql), sg.dev<int32_t>(c, o_cu),
                 sg.dev<uint32_t>(c, o_len), sg.dev<uint32_t>(c, o_ext), sg.dev<uint32_t>(c, o_pages),
                 (float*)c->part_o.p, (float*)c->part_ml.p};
  return attn_enqueue(plan, dp, q, q_dtype == TGOHIP_F16, k, v, out, out_dtype == TGOHIP_F16, T, H,
                      H_kv, max_pages, block, scale, c->stream);
}

// Plans once and replays the launch `iters` times (benchmark helper): the
// metadata stays resident so each replay is the kernels alone.
int tgohip_paged_attention_replay(tgohip_ctx* c, const void* q, int q_dtype, int T, int H, int H_kv,
                                  const void* k, const void* v, int capacity, int B,
                                  const uint32_t* lengths, const uint32_t* extents,
                                  const uint32_t* pages, int max_pages, int block, float scale,
                                  void* out, int out_dtype, int iters) {
  AttnPlan plan;
  int rc = attn_build_plan(T, B, lengths, extents, pages, max_pages, block, capacity, H, H_kv, plan,
                           c->cascade, q_dtype != TGOHIP_F16);
  if (rc) return rc;
  if ((rc = ensure_attn_parts(c, plan.parts))) return rc;
  Stager sg;
  const size_t o_len = sg.add(lengths, (size_t)B * 4);
  const size_t o_ext = sg.add(extents, (size_t)B * 4);
  const size_t o_pages = sg.add(pages, (size_t)B * max_pages * 4);
  const size_t o_cu = sg.add(plan.cu.data(), (size_t)B * 4);
  const size_t o_items = sg.add(plan.items.data(), plan.items.size() * sizeof(AttnItem));
  const size_t o_comb = sg.add(plan.combines.data(), plan.combines.size() * sizeof(AttnCombine));
  const size_t o_seql = sg.add(plan.seqlist.data(), plan.seqlist.size() * sizeof(int32_t));
  if ((rc = sg.upload(c))) return rc;
  AttnDevPlan dp{sg.dev<AttnItem>(c, o_items), sg.dev<AttnCombine>(c, o_comb),
                 sg.dev<int32_t>(c, o_seql), sg.dev<int32_t>(c, o_cu),
                 sg.dev<uint32_t>(c, o_len), sg.dev<uint32_t>(c, o_ext), sg.dev<uint32_t>(c, o_pages),
                 (float*)c->part_o.p, (float*)c->part_ml.p};
  for (int i = 0; i < iters; i++)
    if ((rc = attn_enqueue(plan, dp, q, q_dtype == TGOHIP_F16, k, v, out, out_dtype == TGOHIP_F16, T,
                           H, H_kv, max_pages, block, scale, c->stream)))
      return rc;
  return 0;
}

int tgohip_weight_upload(tgohip_ctx* c, int form, int K, int N, const void* plane,
                         const void* scales, const void* zeros, int* handle) {
  int rc = check_shape(form, K, N, "weight");
  if (rc) return rc;
  Canon cn;
  if ((rc = canon_upload(c, cn, form, K, N, plane, scales, zeros))) return rc;
  PackedWeight w;
  if ((rc = alloc_packed(c, w, form, K, N))) return rc;
  if ((rc = repack_enqueue(form, cn.plane, cn.scales, cn.zeros, K, N, w, 1, 0, c->stream))) return rc;
  TGOHIP_HIP(hipStreamSynchronize(c->stream));
  *handle = c->next_handle++;
  c->handles[*handle] = w;
  return 0;
}

// tgohip_weight_upload from an f32 plane quantized on the device.
int tgohip_weight_upload_f32(tgohip_ctx* c, int form, int K, int N, const float* w, int* handle) {
  int rc = check_shape(form, K, N, "weight");
  if (rc) return rc;
  Canon cn;
  if ((rc = canon_quantize(c, cn, form, K, N, w))) return rc;
  PackedWeight pw;
  if ((rc = alloc_packed(c, pw, form, K, N))) return rc;
  if ((rc = repack_enqueue(form, cn.plane, cn.scales, cn.zeros, K, N, pw, 1, 0, c->stream))) return rc;
  TGOHIP_HIP(hipStreamSynchronize(c->stream));
  *handle = c->next_handle++;
  c->handles[*handle] = pw;
  return 0;
}

// Synthesises a weight on the device under a handle (benchmark shapes).
int tgohip_weight_synth(tgohip_ctx* c, int form, int K, int N, uint64_t seed, uint64_t stream,
                        double sigma, int* handle) {
  int rc = check_shape(form, K, N, "weight");
  if (rc) return rc;
  Canon cn;
  if ((rc = canon_synth(c, cn, seed, stream, form, K, N, sigma))) return rc;
  PackedWeight w;
  if ((rc = alloc_packed(c, w, form, K, N))) return rc;
  if ((rc = repack_enqueue(form, cn.plane, cn.scales, cn.zeros, K, N, w, 1, 0, c->stream))) return rc;
  TGOHIP_HIP(hipStreamSynchronize(c->stream));
  *handle = c->next_handle++;
  c->handles[*handle] = w;
  return 0;
}

int tgohip_weight_free(tgohip_ctx* c, int handle) {
  auto it = c->handles.find(handle);
  if (it == c->handles.end()) return fail(TGOHIP_EINVAL, "weight_free: no handle " + std::to_string(handle));
  TGOHIP_HIP(hipStreamSynchronize(c->stream));
  free_packed(c, it->second);
  c->handles.erase(it);
  return 0;
}

static PackedWeight* handle_of(tgohip_ctx* c, int handle) {
  auto it = c->handles.find(handle);
  if (it == c->handles.end()) {
    fail(TGOHIP_EINVAL, "no weight handle " + std::to_string(handle));
    return nullptr;
  }
  return &it->second;
}

// TGOHIP_F32 / F16 / F16X2 as the kernels' activation kinds.
static int xkind(int x_dtype) {
  return x_dtype == TGOHIP_F32 ? XK_F32 : x_dtype == TGOHIP_F16X2 ? XK_X2 : XK_F16;
}

int tgohip_linear(tgohip_ctx* c, int handle, const void* x, int x_dtype, int M, void* y, int y_dtype) {
  PackedWeight* w = handle_of(c, handle);
  if (!w) return TGOHIP_EINVAL;
  if (M < 0) return fail(TGOHIP_EINVAL, "linear: M is " + std::to_string(M));
  if (M == 0) return 0;  // an empty batch: nothing to launch
  const size_t ws = gemm_workspace_bytes(*w, M, c->ncu);
  int rc = c->gemm_ws.ensure(ws + 256);
  if (rc) return rc;
  return gemm_enqueue(*w, x, xkind(x_dtype), M, y,
                      y_dtype == TGOHIP_F16 ? EPI_F16 : EPI_F32,
                      (float*)c->gemm_ws.p, c->gemm_ws.bytes, c->ncu, c->stream);
}

// tgohip_linear without allocating: the split-K partials go to the static
// `scratch` array (kScratchBytes, this device's copy) instead of the
// context's workspace. Same kernels, same splits, so the same result.
int tgohip_linear_noalloc(tgohip_ctx* c, int handle, const void* x, int x_dtype, int M, void* y,
                          int y_dtype) {
  PackedWeight* w = handle_of(c, handle);
  if (!w) return TGOHIP_EINVAL;
  if (M < 0) return fail(TGOHIP_EINVAL, "linear_noalloc: M is " + std::to_string(M));
  if (M == 0) return 0;  // an empty batch: nothing to launch
  // exactly what this call's kernels use (its activation type decides them)
  const size_t ws = gemm_workspace_bytes(*w, M, c->ncu, xkind(x_dtype));
  if (ws > kScratchBytes)
    return fail(TGOHIP_EINVAL, "linear_noalloc: M = " + std::to_string(M) + " over [" +
                                   std::to_string(w->K) + "," + std::to_string(w->N) +
                                   "] needs " + std::to_string(ws) + " bytes of split-K partials "
                                   "and the static workspace holds " +
                                   std::to_string(kScratchBytes) + "; use tgohip_linear");
  if (!c->scratch) return fail(TGOHIP_ESTATE, "linear_noalloc: no workspace address for this device");
  return gemm_enqueue(*w, x, xkind(x_dtype), M, y,
                      y_dtype == TGOHIP_F16 ? EPI_F16 : EPI_F32,
                      (float*)c->scratch, kScratchBytes, c->ncu, c->stream);
}

int tgohip_linear_workspace(tgohip_ctx* c, int handle, int x_dtype, int M, size_t* bytes) {
  PackedWeight* w = handle_of(c, handle);
  if (!w) return TGOHIP_EINVAL;
  if (M < 0) return fail(TGOHIP_EINVAL, "linear_workspace: M is " + std::to_string(M));
  *bytes = gemm_workspace_bytes(*w, M, c->ncu, xkind(x_dtype));
  return 0;
}

int tgohip_dequant(tgohip_ctx* c, int handle, float* y) {
  PackedWeight* w = handle_of(c, handle);
  if (!w) return TGOHIP_EINVAL;
  return dequant_enqueue(*w, y, false, c->stream);
}

int tgohip_dequant_f16(tgohip_ctx* c, int handle, uint16_t* y) {
  PackedWeight* w = handle_of(c, handle);
  if (!w) return TGOHIP_EINVAL;
  return dequant_enqueue(*w, y, true, c->stream);
}

}  // extern "C"

// ===========================================================================
// Scheduler: scheduler.go + Batch (batch.go) over the prefix pool
// ===========================================================================
struct SchedSlot {
  bool live = false;
  std::vector<int32_t> prompt;
  int prefilled = 0;
  int feed = 0;
  int reused = 0;
  uint64_t arrived = 0;
  PrefixLease* lease = nullptr;
  std::vector<int> pages;
  int length = 0;
  // Overlap mode: the books projected past the steps in flight (prompt length
  // counting generated tokens not yet read back, positions scored, length).
  int plen_p = 0, pf_p = 0, len_p = 0;
  int inflight = 0;       // steps in flight holding rows of this slot
  bool pending = false;   // its next row's token is its entry of the device argmax
  bool retiring = false;  // finished while rows were in flight: released when they land
};

// A step submitted in overlap mode and not yet collected.
struct InflightStep {
  std::vector<int> ws, wst, wc;  // working slots, prompt start (-1: decode row), rows
  std::vector<int> row0;         // each working slot's first row
  std::vector<char> done;        // the slot's prompt is scored once the step lands
  int parity = 0;
  int32_t prefill = 0, decodes = 0;
  double submit_ms = 0;
  ProfStep prof;
};

static void sync_proj(SchedSlot& s) {
  s.plen_p = (int)s.prompt.size();
  s.pf_p = s.prefilled;
  s.len_p = s.length;
}

struct tgohip_sched {
  tgohip_ctx* ctx;
  int chunk, reserve, max_rows;
  std::unique_ptr<PrefixPool> pool;
  std::vector<SchedSlot> slots;
  uint64_t next = 0;
  // reusable host buffers
  std::vector<uint32_t> ids, posq, posk, slotv, lengths, extents, last, table;
  int table_stride = 1;  // row stride of table: the longest lease of the last step
  std::vector<int32_t> argmax;
  // overlap mode (tgohip_sched_set_overlap)
  bool overlap = false;
  std::deque<InflightStep> flight;
  int parity = 0;
  hipEvent_t ev[2][3] = {};        // per parity: begin, kernels done, argmax copied
  int32_t* amax_host[2] = {};      // per parity: pinned copy of the step's argmax
};

static void slot_release(SchedSlot& s) {
  if (s.lease) {
    s.lease->release();
    delete s.lease;
    s.lease = nullptr;
  }
  s.pages.clear();
}

extern "C" {

tgohip_sched* tgohip_sched_new(tgohip_ctx* c, int n, int chunk, int reserve, int max_rows) {
  if (reserve <= 0) {
    fail(TGOHIP_EINVAL, "the scheduler's reserve is " + std::to_string(reserve) +
                            "; it is how many positions an admitted sequence may grow by, and "
                            "admitting without one fills every slot with sequences that cannot grow");
    return nullptr;
  }
  if (chunk == 0) chunk = 512;  // DefaultChunk (schedule.go:21)
  if (chunk < 0) {
    fail(TGOHIP_EINVAL, "the prefill chunk is " + std::to_string(chunk) + "; a chunk is at least one token");
    return nullptr;
  }
  if (n < 2) {
    fail(TGOHIP_EINVAL, "a batch of " + std::to_string(n) + " slot(s) is a session; a batch is two or more");
    return nullptr;
  }
  if (!c->kc) {
    fail(TGOHIP_ESTATE, "a batched step needs a shared block pool");
    return nullptr;
  }
  auto* s = new tgohip_sched();
  s->ctx = c;
  s->chunk = chunk;
  s->reserve = reserve;
  s->max_rows = max_rows > 0 ? max_rows : c->kv_positions;
  s->pool.reset(new PrefixPool(c->cfg.block, c->kv_positions / c->cfg.block, 0));
  s->slots.resize(n);
  return s;
}

void tgohip_sched_free(tgohip_sched* s) {
  if (!s) return;
  if (!s->flight.empty()) (void)hipStreamSynchronize(s->ctx->stream);
  for (auto& sl : s->slots) slot_release(sl);
  for (int p = 0; p < 2; p++) {
    for (hipEvent_t& e : s->ev[p])
      if (e) (void)hipEventDestroy(e);
    if (s->amax_host[p]) (void)hipHostFree(s->amax_host[p]);
  }
  delete s;
}

int tgohip_sched_admit(tgohip_sched* s, const int32_t* prompt, int n, int reserve) {
  if (reserve == 0) reserve = s->reserve;
  if (reserve < 0) return fail(TGOHIP_EINVAL, "the reserve is " + std::to_string(reserve));
  if (n <= 0) return fail(TGOHIP_EINVAL, "the prompt is empty; there is nothing to condition on");
  int free = -1;
  for (int i = 0; i < (int)s->slots.size(); i++)
    if (!s->slots[i].live && s->slots[i].inflight == 0) { free = i; break; }
  if (free < 0) return fail(TGOHIP_ENOSLOT, "every slot is occupied");
  SchedSlot& sl = s->slots[free];
  slot_release(sl);
  PrefixLease* l = nullptr;
  int rc = s->pool->acquire(prompt, n, "", "", reserve, &l);
  if (rc) return rc;
  sl.lease = l;
  sl.pages = l->blocks;
  sl.length = l->reused;
  s->next++;
  sl.live = true;
  sl.prompt.assign(prompt, prompt + n);
  sl.prefilled = l->reused;
  sl.reused = l->reused;
  sl.arrived = s->next;
  sl.feed = 0;
  sync_proj(sl);
  return free;
}

int tgohip_sched_finish(tgohip_sched* s, int slot) {
  if (slot < 0 || slot >= (int)s->slots.size())
    return fail(TGOHIP_EINVAL, "slot " + std::to_string(slot) + " is outside a batch of " +
                                   std::to_string(s->slots.size()));
  SchedSlot& sl = s->slots[slot];
  if (sl.inflight > 0) {
    // rows of it are still in flight (overlap mode): they land first
    sl.live = false;
    sl.retiring = true;
    return 0;
  }
  slot_release(sl);
  sl = SchedSlot();
  return 0;
}

int tgohip_sched_evict(tgohip_sched* s) {
  std::vector<int32_t> live, plen, pf;
  std::vector<uint64_t> arr;
  for (auto& sl : s->slots) {
    live.push_back(sl.live);
    plen.push_back((int32_t)sl.prompt.size());
    pf.push_back(sl.prefilled);
    arr.push_back(sl.arrived);
  }
  const int v = tgohip_victim((int)s->slots.size(), live.data(), plen.data(), pf.data(), arr.data());
  if (v < 0) return -1;
  tgohip_sched_finish(s, v);
  return v;
}

int tgohip_sched_feed(tgohip_sched* s, int slot, int token) {
  if (slot < 0 || slot >= (int)s->slots.size())
    return fail(TGOHIP_EINVAL, "slot " + std::to_string(slot) + " is outside a batch of " +
                                   std::to_string(s->slots.size()));
  SchedSlot& sl = s->slots[slot];
  if (!sl.live) return fail(TGOHIP_EINVAL, "slot " + std::to_string(slot) + " holds no sequence");
  if (sl.pending || sl.inflight > 0)
    return fail(TGOHIP_ESTATE, "slot " + std::to_string(slot) + " has rows in flight or is fed "
                               "by the device: in overlap mode the scheduler feeds each generated "
                               "token itself");
  if (sl.prefilled < (int)sl.prompt.size())
    return fail(TGOHIP_EINVAL, "slot " + std::to_string(slot) + " is " + std::to_string(sl.prefilled) +
                                   " tokens into a " + std::to_string(sl.prompt.size()) +
                                   "-token prompt; a token fed before the prompt is scored would be "
                                   "generated from a distribution over the middle of it");
  if (token < 0 || token >= s->ctx->cfg.vocab)
    return fail(TGOHIP_EINVAL, "token id " + std::to_string(token) +
                                   " is outside the model's vocabulary of " + std::to_string(s->ctx->cfg.vocab));
  sl.feed = token;
  sl.prompt.push_back(token);
  sl.prefilled++;
  sync_proj(sl);
  return 0;
}

int tgohip_sched_length(tgohip_sched* s, int slot) {
  if (slot < 0 || slot >= (int)s->slots.size()) return 0;
  return s->slots[slot].length;
}

int tgohip_sched_step(tgohip_sched* s, int32_t* out_slot, int32_t* out_token, int32_t* out_done,
                      int32_t* prefill_tokens, int32_t* decodes, tgohip_timings* tm) {
  if (s->overlap)
    return fail(TGOHIP_ESTATE, "the scheduler is in overlap mode: steps go through "
                               "tgohip_sched_submit and tgohip_sched_collect");
  const int n = (int)s->slots.size();
  const tgohip_model_cfg& m = s->ctx->cfg;
  std::vector<int32_t> live(n), plen(n), pf(n), ws(n), wst(n), wc(n);
  for (int i = 0; i < n; i++) {
    live[i] = s->slots[i].live;
    plen[i] = (int32_t)s->slots[i].prompt.size();
    pf[i] = s->slots[i].prefilled;
  }
  int32_t nw = 0, npf = 0, ndc = 0;
  int rc = tgohip_next_step(n, live.data(), plen.data(), pf.data(), s->chunk, s->max_rows, ws.data(),
                            wst.data(), wc.data(), &nw, &npf, &ndc);
  if (rc) return rc;
  *prefill_tokens = npf;
  *decodes = ndc;
  if (nw == 0) return 0;
  // Batch.step: every slot is a member; workers reserve blocks first.
  std::vector<int32_t> counts(n, 0), first(n, 0), toks;
  std::vector<std::vector<int32_t>> wtok(n);
  for (int i = 0; i < nw; i++) {
    const int sl = ws[i];
    SchedSlot& st = s->slots[sl];
    if (wst[i] >= 0) wtok[sl].assign(st.prompt.begin() + wst[i], st.prompt.begin() + wst[i] + wc[i]);
    else wtok[sl] = {st.feed};
    const int need = st.length + (int)wtok[sl].size();
    if (need > (int)st.lease->ids.size()) {
      if ((rc = st.lease->grow(need - (int)st.lease->ids.size()))) return rc;
    }
    st.pages = st.lease->blocks;
  }
  int total = 0, maxp = 1;
  for (int i = 0; i < n; i++) {
    first[i] = s->slots[i].length;
    counts[i] = (int32_t)wtok[i].size();
    total += counts[i];
    maxp = std::max(maxp, (int)s->slots[i].pages.size());
    toks.insert(toks.end(), wtok[i].begin(), wtok[i].end());
  }
  // The table's row stride is the longest lease of the step, not the whole
  // pool (batch.go sizes it by the pool; only the stride differs, every row
  // is still zero past its lease). At C4 this is ~600 entries instead of
  // 25,000: the table shrinks from 13.6 MB to ~0.3 MB per step.
  const int maxPages = maxp;
  std::vector<int32_t> pagesv((size_t)n * maxPages, 0), plens(n, 0);
  s->table_stride = maxPages;
  s->table.assign((size_t)n * maxPages, 0u);
  for (int i = 0; i < n; i++) {
    plens[i] = (int32_t)s->slots[i].pages.size();
    for (size_t j = 0; j < s->slots[i].pages.size(); j++) {
      pagesv[(size_t)i * maxPages + j] = s->slots[i].pages[j];
      s->table[(size_t)i * maxPages + j] = (uint32_t)s->slots[i].pages[j];
    }
  }
  const int rows = total;
  s->ids.resize(rows);
  s->posq.resize((size_t)rows * m.heads);
  s->posk.resize((size_t)rows * m.kv_heads);
  s->slotv.resize(rows);
  s->lengths.resize(n);
  s->extents.resize(n);
  s->last.resize(n);
  s->argmax.resize(n);
  rc = tgohip_new_batch_step(m.vocab, m.heads, m.kv_heads, rows, n, toks.data(), counts.data(),
                             first.data(), pagesv.data(), plens.data(), maxPages, m.block,
                             s->ctx->kv_positions, s->ids.data(), s->posq.data(), s->posk.data(),
                             s->slotv.data(), s->lengths.data(), s->extents.data(), s->last.data());
  if (rc) return rc;
  tgohip_batch_step bs{rows, n, maxPages, s->ids.data(), s->posq.data(), s->posk.data(),
                       s->slotv.data(), s->lengths.data(), s->extents.data(), s->last.data(),
                       s->table.data()};
  if ((rc = tgohip_step(s->ctx, &bs, nullptr, s->argmax.data(), tm))) return rc;
  // commit: the step landed (batch.go:443-456), then the scheduler's books.
  int produced = 0;
  for (int i = 0; i < nw; i++) {
    const int sl = ws[i];
    SchedSlot& st = s->slots[sl];
    const std::vector<int32_t>& tk = wtok[sl];
    const int need = st.length + (int)tk.size();
    if (need > (int)st.lease->ids.size()) {
      const int extra = need - (int)st.lease->ids.size();
      if ((rc = st.lease->commit(tk.data() + tk.size() - extra, extra))) return rc;
    }
    st.lease->publish(st.length + (int)tk.size());
    st.pages = st.lease->blocks;
    st.length += (int)tk.size();
    const bool prefill = st.prefilled < (int)st.prompt.size();
    if (prefill) st.prefilled += (int)tk.size();
    sync_proj(st);
    out_slot[produced] = sl;
    out_token[produced] = s->argmax[sl];
    out_done[produced] = st.prefilled >= (int)st.prompt.size();
    produced++;
  }
  return produced;
}

// ---- overlap mode: the next step is submitted before the last is read back
//
// tgo's Batch.step packs, uploads, submits, waits and reads back in one call
// under the model's lock (batch.go:381-437): the device idles while the host
// schedules. Here submit() enqueues a step and returns at once, and collect()
// waits for the oldest step in flight and commits it. A decode row's token is
// the previous step's argmax, read on the device (the argmax array keeps each
// slot's latest token), so step k+1 can be submitted before step k is read
// back. posq/posk/slots are derived on the device from the members' lengths,
// extents and page rows, so only ids and the per-member ports cross PCIe. The
// staging buffers and events alternate between two sets.
int tgohip_sched_set_overlap(tgohip_sched* s, int on) {
  if (!s->flight.empty())
    return fail(TGOHIP_ESTATE, "steps are in flight; collect them before switching modes");
  if (on && !s->ev[0][0]) {
    for (int p = 0; p < 2; p++) {
      // begin and kernels-done mark timing only; the third (argmax copied)
      // precedes a host read and keeps the system-scope fence
      TGOHIP_HIP(hipEventCreateWithFlags(&s->ev[p][0], hipEventDisableSystemFence));
      TGOHIP_HIP(hipEventCreateWithFlags(&s->ev[p][1], hipEventDisableSystemFence));
      TGOHIP_HIP(hipEventCreate(&s->ev[p][2]));
      TGOHIP_HIP(hipHostMalloc((void**)&s->amax_host[p], s->slots.size() * 4, hipHostMallocDefault));
    }
  }
  if (on && !s->overlap) {
    for (auto& sl : s->slots) {
      if (sl.live && sl.prefilled >= (int)sl.prompt.size() && sl.length >= (int)sl.prompt.size()) {
        // a decoding slot whose last token the caller fed: the host holds it
        sl.pending = false;
      }
      sync_proj(sl);
    }
  }
  if (!on && s->overlap) {
    // back to host feeding: each device-fed slot's token is its last history entry
    for (auto& sl : s->slots) sl.pending = false;
  }
  s->overlap = on != 0;
  return 0;
}

int tgohip_sched_submit(tgohip_sched* s, int32_t* out_slot, int32_t* out_done,
                        int32_t* prefill_tokens, int32_t* decodes) {
  using clk = std::chrono::steady_clock;
  const auto t0 = clk::now();
  if (!s->overlap) return fail(TGOHIP_ESTATE, "submit needs overlap mode (tgohip_sched_set_overlap)");
  if (s->flight.size() >= 2)
    return fail(TGOHIP_ESTATE, "two steps are in flight; collect one before submitting another");
  tgohip_ctx* c = s->ctx;
  const int n = (int)s->slots.size();
  std::vector<int32_t> live(n), plen(n), pf(n), ws(n), wst(n), wc(n);
  for (int i = 0; i < n; i++) {
    const SchedSlot& sl = s->slots[i];
    live[i] = sl.live;
    plen[i] = sl.plen_p;
    pf[i] = sl.pf_p;
  }
  int32_t nw = 0, npf = 0, ndc = 0;
  int rc = tgohip_next_step(n, live.data(), plen.data(), pf.data(), s->chunk, s->max_rows, ws.data(),
                            wst.data(), wc.data(), &nw, &npf, &ndc);
  if (rc) return rc;
  *prefill_tokens = npf;
  *decodes = ndc;
  if (nw == 0) return 0;
  InflightStep f;
  f.parity = s->parity;
  f.prefill = npf;
  f.decodes = ndc;
  std::vector<int32_t> counts(n, 0);
  std::vector<uint32_t> rowid;  // ids in member order
  std::vector<std::vector<uint32_t>> wid(n);
  for (int i = 0; i < nw; i++) {
    const int sl = ws[i];
    SchedSlot& st = s->slots[sl];
    if (wst[i] >= 0) {
      if (wst[i] + wc[i] > (int)st.prompt.size())
        return fail(TGOHIP_ESTATE, "slot " + std::to_string(sl) + ": a prompt chunk reaches past "
                                   "the tokens the host holds");
      for (int j = 0; j < wc[i]; j++) wid[sl].push_back((uint32_t)st.prompt[wst[i] + j]);
    } else {
      wid[sl].push_back(st.pending ? (0x80000000u | (uint32_t)sl) : (uint32_t)st.feed);
    }
    const int need = st.len_p + (int)wid[sl].size();
    if (need > (int)st.lease->ids.size()) {
      if ((rc = st.lease->grow(need - (int)st.lease->ids.size()))) return rc;
    }
    st.pages = st.lease->blocks;
  }
  int total = 0, maxp = 1;
  for (int i = 0; i < n; i++) {
    counts[i] = (int32_t)wid[i].size();
    total += counts[i];
    maxp = std::max(maxp, (int)s->slots[i].pages.size());
  }
  s->table_stride = maxp;
  s->table.assign((size_t)n * maxp, 0u);
  s->ids.resize(total);
  s->lengths.resize(n);
  s->extents.resize(n);
  s->last.resize(n);
  s->posq.clear();
  s->posk.clear();
  s->slotv.clear();
  int at = 0;
  std::vector<int> row0(n, 0);
  for (int i = 0; i < n; i++) {
    const SchedSlot& st = s->slots[i];
    row0[i] = at;
    for (size_t j = 0; j < st.pages.size(); j++) s->table[(size_t)i * maxp + j] = (uint32_t)st.pages[j];
    s->lengths[i] = (uint32_t)(st.len_p + counts[i]);
    s->extents[i] = (uint32_t)counts[i];
    s->last[i] = counts[i] > 0 ? (uint32_t)(at + counts[i] - 1) : 0u;
    for (uint32_t id : wid[i]) s->ids[at++] = id;
  }
  tgohip_batch_step bs{total, n, maxp, s->ids.data(), nullptr, nullptr, nullptr,
                       s->lengths.data(), s->extents.data(), s->last.data(), s->table.data()};
  if ((rc = ensure_activations(c, total, n))) return rc;  // argmax holds n entries from here
  StepLaunch o;
  o.feed = (const int32_t*)c->argmax.p;
  o.keep_idle = 1;
  o.ev_begin = s->ev[f.parity][0];
  o.ev_end = s->ev[f.parity][1];
  o.prof_set = f.parity;
  if ((rc = step_launch(c, &bs, o))) return rc;
  TGOHIP_HIP(hipMemcpyAsync(s->amax_host[f.parity], c->argmax.p, (size_t)n * 4,
                            hipMemcpyDeviceToHost, c->stream));
  TGOHIP_HIP(hipEventRecord(s->ev[f.parity][2], c->stream));
  f.prof = o.prof;
  // the books as they will stand once this step lands
  int produced = 0;
  for (int i = 0; i < nw; i++) {
    const int sl = ws[i];
    SchedSlot& st = s->slots[sl];
    st.len_p += counts[sl];
    st.inflight++;
    if (wst[i] >= 0) st.pf_p += wc[i];
    const bool gen = st.pf_p >= st.plen_p;
    if (gen) {  // the step generates a token, fed to the slot's next row
      st.plen_p++;
      st.pf_p++;
      st.pending = true;
    }
    f.ws.push_back(sl);
    f.wst.push_back(wst[i]);
    f.wc.push_back(counts[sl]);
    f.row0.push_back(row0[sl]);
    f.done.push_back(gen ? 1 : 0);
    out_slot[produced] = sl;
    out_done[produced] = gen ? 1 : 0;
    produced++;
  }
  f.submit_ms = std::chrono::duration<double, std::milli>(clk::now() - t0).count();
  s->flight.push_back(std::move(f));
  s->parity ^= 1;
  return produced;
}

int tgohip_sched_collect(tgohip_sched* s, int32_t* out_slot, int32_t* out_token, int32_t* out_done,
                         tgohip_timings* tm) {
  if (s->flight.empty()) return 0;
  InflightStep& f = s->flight.front();
  TGOHIP_HIP(hipEventSynchronize(s->ev[f.parity][2]));
  const int32_t* amax = s->amax_host[f.parity];
  int rc = 0;
  int produced = 0;
  for (size_t i = 0; i < f.ws.size(); i++) {
    const int sl = f.ws[i];
    SchedSlot& st = s->slots[sl];
    // the rows' tokens: a prompt chunk, or the slot's fed token (one the
    // device fed was recorded when the step before was collected)
    std::vector<int32_t> tk;
    if (f.wst[i] >= 0) tk.assign(st.prompt.begin() + f.wst[i], st.prompt.begin() + f.wst[i] + f.wc[i]);
    else tk.push_back(st.feed);
    // the last step submitted keeps its ports (tgohip_sched_last_step): a
    // device-fed id becomes the token it stood for
    if (s->flight.size() == 1 && f.wst[i] < 0) s->ids[f.row0[i]] = (uint32_t)st.feed;
    const int need = st.length + (int)tk.size();
    if (need > (int)st.lease->ids.size()) {
      const int extra = need - (int)st.lease->ids.size();
      if ((rc = st.lease->commit(tk.data() + tk.size() - extra, extra))) {
        s->flight.pop_front();  // the step landed; its books cannot be completed
        return rc;
      }
    }
    st.lease->publish(st.length + (int)tk.size());
    st.pages = st.lease->blocks;
    st.length += (int)tk.size();
    if (st.prefilled < (int)st.prompt.size()) st.prefilled += (int)tk.size();
    const int tok = amax[sl];
    if (f.done[i]) {  // the generated token joins the history (the device fed it already)
      st.feed = tok;
      st.prompt.push_back(tok);
      st.prefilled++;
    }
    out_slot[produced] = sl;
    out_token[produced] = tok;
    out_done[produced] = f.done[i];
    produced++;
    st.inflight--;
    if (st.retiring && st.inflight == 0) {
      slot_release(st);
      st = SchedSlot();
    }
  }
  if ((rc = profile_collect(s->ctx, f.parity, f.prof))) return rc;
  if (tm) {
    float dev_ms = 0;
    (void)hipEventElapsedTime(&dev_ms, s->ev[f.parity][0], s->ev[f.parity][1]);
    tm->submit_ms = f.submit_ms;
    tm->device_ms = dev_ms;
    tm->readback_ms = 0;
  }
  s->flight.pop_front();
  return produced;
}

}  // extern "C"

// ===========================================================================
// measurement and benchmark helpers
// ===========================================================================
extern "C" {

int tgohip_set_profile_kernels(tgohip_ctx* c, int stride, int mask) {
  if (stride < 0) return fail(TGOHIP_EINVAL, "profile: " + std::to_string(stride) + " is not a layer stride");
  if (mask < 0 || mask >= (1 << TGOHIP_PROF_KINDS))
    return fail(TGOHIP_EINVAL, "profile: kernel mask " + std::to_string(mask) + " names no kernel kinds");
  c->profile = stride != 0 && mask != 0;
  c->prof_stride = stride > 0 ? stride : 1;
  c->prof_mask = mask;
  for (int k = 0; k < TGOHIP_PROF_KINDS; k++) {
    c->prof_ms[k] = c->prof_bytes[k] = c->prof_flops[k] = 0;
    c->prof_launches[k] = 0;
  }
  return 0;
}

int tgohip_set_profile(tgohip_ctx* c, int on) {
  return tgohip_set_profile_kernels(c, on, 1 << TGOHIP_PROF_ATTN);
}

int tgohip_profile_read_kernel(tgohip_ctx* c, int kind, double* ms, double* bytes, double* flops,
                               int64_t* launches) {
  if (kind < 0 || kind >= TGOHIP_PROF_KINDS)
    return fail(TGOHIP_EINVAL, "profile: no kernel kind " + std::to_string(kind));
  *ms = c->prof_ms[kind];
  *bytes = c->prof_bytes[kind];
  *flops = c->prof_flops[kind];
  *launches = c->prof_launches[kind];
  return 0;
}

int tgohip_profile_read(tgohip_ctx* c, double* attn_ms, double* attn_bytes, int64_t* launches) {
  double flops = 0;
  return tgohip_profile_read_kernel(c, TGOHIP_PROF_ATTN, attn_ms, attn_bytes, &flops, launches);
}

// The box's achievable peaks: a streaming read of read_bytes (a buffer this
// call allocates, fills and frees) and a dense f16 MFMA loop over every CU;
// medians of reps timed launches on the context's stream, after one untimed.
int tgohip_probe_peaks(tgohip_ctx* c, size_t read_bytes, int reps, double* read_gbps,
                       double* mfma_tflops) {
  if (read_bytes < ((size_t)1 << 20) || reps < 1)
    return fail(TGOHIP_EINVAL, "probe_peaks: read_bytes " + std::to_string(read_bytes) +
                                   " (at least 1 MiB) and reps " + std::to_string(reps) +
                                   " (at least 1)");
  read_bytes &= ~(size_t)15;
  void* buf = nullptr;
  void* sink = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  std::vector<float> rt, mt;
  double flops = 0;
  int rc = 0;
  auto cleanup = [&] {
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (buf) (void)hipFree(buf);
    if (sink) (void)hipFree(sink);
  };
  if (hipMalloc(&buf, read_bytes) != hipSuccess || hipMalloc(&sink, 256) != hipSuccess ||
      hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    cleanup();
    return fail(TGOHIP_ENOMEM, "probe_peaks: " + std::to_string(read_bytes) + " bytes");
  }
  auto timed = [&](auto launch, std::vector<float>& out) -> int {
    for (int i = 0; i <= reps; i++) {
      if (hipEventRecord(e0, c->stream) != hipSuccess) return fail(TGOHIP_EDEVICE, "probe: event");
      int r = launch();
      if (r) return r;
      if (hipEventRecord(e1, c->stream) != hipSuccess || hipEventSynchronize(e1) != hipSuccess)
        return fail(TGOHIP_EDEVICE, "probe: event");
      float ms = 0;
      if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) return fail(TGOHIP_EDEVICE, "probe: timing");
      if (i > 0) out.push_back(ms);
    }
    std::sort(out.begin(), out.end());
    return 0;
  };
  if (hipMemsetAsync(buf, 0x5a, read_bytes, c->stream) != hipSuccess) rc = fail(TGOHIP_EDEVICE, "probe: fill");
  if (!rc)
    rc = timed([&] { return probe_read_enqueue(buf, read_bytes, (uint32_t*)sink, c->stream); }, rt);
  if (!rc)
    rc = timed([&] {
      flops = probe_mfma_enqueue(4 * c->ncu, 2048, (float*)sink, c->stream);
      return (int)(hipGetLastError() != hipSuccess ? fail(TGOHIP_EDEVICE, "probe: mfma launch") : 0);
    }, mt);
  cleanup();
  if (rc) return rc;
  *read_gbps = read_bytes / (rt[rt.size() / 2] * 1e-3) / 1e9;
  *mfma_tflops = flops / (mt[mt.size() / 2] * 1e-3) / 1e12;
  return 0;
}

// Fills positions [0, positions) of every layer of the K and V pools with
// loader-rule f16 of N(0,1)*sigma from (seed, stream 0x4b / 0x56): the synthetic
// context of sequences admitted already prefilled.
int tgohip_kv_synth(tgohip_ctx* c, uint64_t seed, double sigma, int positions) {
  if (!c->kc) return fail(TGOHIP_ESTATE, "kv_synth: allocate the pool first");
  positions = std::min(positions, c->kv_positions);
  const size_t row = (size_t)c->cfg.kv_heads * kHeadDim;
  for (int l = 0; l < c->cfg.layers; l++) {
    const size_t off = (size_t)l * c->kv_positions * row;
    // one stream per layer so a layer's contents do not depend on the pool size
    launch_synth_f16(seed, 0x4b00 + (uint64_t)l, (size_t)positions * row, sigma,
                     (uint16_t*)(c->kc + off), c->stream);
    launch_synth_f16(seed, 0x5600 + (uint64_t)l, (size_t)positions * row, sigma,
                     (uint16_t*)(c->vc + off), c->stream);
  }
  TGOHIP_HIP(hipGetLastError());
  TGOHIP_HIP(hipStreamSynchronize(c->stream));
  return 0;
}

// Admits a sequence whose prompt's KV is already in the pool (restored or
// synthetic): the lease covers the prompt and the slot starts decoding, its
// first fed token being `feed`.
int tgohip_sched_admit_prefilled(tgohip_sched* s, const int32_t* prompt, int n, int reserve,
                                 int feed) {
  const int slot = tgohip_sched_admit(s, prompt, n, reserve);
  if (slot < 0) return slot;
  SchedSlot& sl = s->slots[slot];
  sl.prefilled = n;
  sl.length = n;
  sl.feed = feed;
  // The prompt's KV is in place: its whole blocks are published, as a
  // prefill would have published them, so later prompts that begin alike
  // share them (publishing may adopt an identical block already cached).
  sl.lease->publish(n);
  sl.pages = sl.lease->blocks;
  sync_proj(sl);
  return slot;
}

// Sequences still being prefilled; in overlap mode, once the steps in flight
// have landed.
int tgohip_sched_prefilling(tgohip_sched* s) {
  int k = 0;
  for (auto& sl : s->slots)
    if (sl.live && sl.pf_p < sl.plen_p) k++;
  return k;
}

int tgohip_sched_live(tgohip_sched* s) {
  int k = 0;
  for (auto& sl : s->slots) k += sl.live ? 1 : 0;
  return k;
}

// The ports of the scheduler's last step (for replaying it elsewhere, e.g. on
// the CPU restatement). Pass NULL arrays to learn the sizes first.
int tgohip_sched_last_step(tgohip_sched* s, int32_t* rows, int32_t* batch, int32_t* max_pages,
                           uint32_t* ids, uint32_t* posq, uint32_t* posk, uint32_t* slots,
                           uint32_t* lengths, uint32_t* extents, uint32_t* last, uint32_t* pages) {
  if (!s->flight.empty())
    return fail(TGOHIP_ESTATE, "last step: a step is in flight; its ids name device tokens "
                               "until it is collected");
  *rows = (int32_t)s->ids.size();
  *batch = (int32_t)s->lengths.size();
  *max_pages = s->table_stride;
  if (s->posq.empty() && !s->ids.empty()) {
    // an overlap-mode step left these to the device: derive them as it did
    const tgohip_model_cfg& m = s->ctx->cfg;
    const int T = (int)s->ids.size(), B = (int)s->lengths.size();
    s->posq.assign((size_t)T * m.heads, 0u);
    s->posk.assign((size_t)T * m.kv_heads, 0u);
    s->slotv.assign(T, 0u);
    int t = 0;
    for (int b = 0; b < B; b++)
      for (uint32_t j = 0; j < s->extents[b]; j++, t++) {
        const uint32_t p = s->lengths[b] - s->extents[b] + j;
        s->slotv[t] = s->table[(size_t)b * s->table_stride + p / m.block] * (uint32_t)m.block +
                      p % (uint32_t)m.block;
        for (int h = 0; h < m.heads; h++) s->posq[(size_t)t * m.heads + h] = p;
        for (int h = 0; h < m.kv_heads; h++) s->posk[(size_t)t * m.kv_heads + h] = p;
      }
  }
  auto cp = [](uint32_t* dst, const std::vector<uint32_t>& v) {
    if (dst) std::memcpy(dst, v.data(), v.size() * 4);
  };
  cp(ids, s->ids);
  cp(posq, s->posq);
  cp(posk, s->posk);
  cp(slots, s->slotv);
  cp(lengths, s->lengths);
  cp(extents, s->extents);
  cp(last, s->last);
  cp(pages, s->table);
  return 0;
}

}  // extern "C"
