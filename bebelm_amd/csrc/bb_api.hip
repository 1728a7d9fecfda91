// bb_api.hip — the C ABI (include/bebelm_moe.h): contexts, HBM-resident weights, and the
// host-side sequencing of the kernels in the order the reference's model.rs issues them.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <exception>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/bebelm_moe.h"
#include "bb_internal.h"

namespace {

thread_local std::string g_err;

struct Fail {
  int code;
};

[[noreturn]] void fail(int code, const std::string& msg) {
  g_err = msg;
  throw Fail{code};
}

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) fail(BB_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

template <class F>
int guard(F&& f) {
  try {
    g_err.clear();
    f();
    return BB_OK;
  } catch (const Fail& x) {
    return x.code;
  } catch (const std::bad_alloc&) {
    g_err = "host allocation failed";
    return BB_ERR_OOM;
  } catch (const std::exception& x) {
    g_err = x.what();
    return BB_ERR_ARG;
  } catch (...) {
    g_err = "unknown error";
    return BB_ERR_ARG;
  }
}

bool block_of(uint32_t dt, size_t& elems, size_t& bytes) {  // tensor.rs:68-93
  switch (dt) {
    case BB_F32: elems = 1; bytes = 4; return true;
    case BB_F16: elems = 1; bytes = 2; return true;
    case BB_Q4_K: elems = 256; bytes = 144; return true;
    case BB_Q6_K: elems = 256; bytes = 210; return true;
    default: return false;
  }
}

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Tail padding behind every device allocation: the Q6_K loader reads whole dwords around
// 2-byte-aligned fields, up to one dword past a block's last byte.
constexpr size_t PAD = 256;

void* dev_alloc(size_t bytes) {
  void* p = nullptr;
  if (hipMalloc(&p, round_up(bytes, 256) + PAD) != hipSuccess) {
    (void)hipGetLastError();
    fail(BB_ERR_OOM, "hipMalloc of " + std::to_string(bytes) + " bytes failed");
  }
  return p;
}


}  // namespace

void bb::set_last_error(const std::string& msg) { g_err = msg; }

// Workspace of bb_moe_forward_noalloc: a fixed area in the code object's static device memory,
// one copy per GPU, held until the process ends. Host code never uses the name `scratch` as an
// address (on the host it only names the symbol): each device's address comes from
// hipGetSymbolAddress at context creation and is kept in g_scratch.
static __device__ __align__(256) uint8_t scratch[BB_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int SCRATCH_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch[SCRATCH_MAX_DEVICES] = {};  // per device, set once under g_scratch_mu

uint8_t* scratch_of(int device) {
  if (device < 0 || device >= SCRATCH_MAX_DEVICES) return nullptr;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  return g_scratch[device];
}
}  // namespace

struct bb_ctx {
  int device = 0;
  hipStream_t own = nullptr;
  hipStream_t stream = nullptr;
  uint8_t* ws = nullptr;
  size_t ws_bytes = 0;
  uint8_t* io = nullptr;  // staging for host-pointer calls
  size_t io_bytes = 0;
  bool profile = false;
  struct Pending {
    int id;
    hipEvent_t a, b;
  };
  std::vector<Pending> pending;
  std::vector<hipEvent_t> event_pool;
  double kernel_ms[bb::K_COUNT] = {};
  int64_t launches[bb::K_COUNT] = {};
  size_t batched_min_entries = 64;  // T*k from which MoE calls take the grouped-GEMM path
  int n_cu = 256;                   // compute units of the device
};

struct bb_tensor {
  bb_ctx* ctx;
  uint32_t dtype;
  uint64_t dims[4];
  int ndims;
  size_t nbytes;
  uint8_t* dev;
};

struct bb_moe {
  bb_ctx* ctx;
  float* bias_dev;
  float* router_cm;    // router regrouped by dot chain (layout of k_route's loads)
  uint8_t* gu_packed;  // gate/up experts, tile-packed and interleaved
  uint8_t* dn_packed;  // down experts, tile-packed
  int H, F, E, K;
  int gu_dtype, dn_dtype;
  size_t stride_gu, stride_dn;  // packed bytes per expert
};

struct bb_dense {
  bb_ctx* ctx;
  const bb_tensor *gate, *up, *down;
  int H, F;
  bb::PackedW gu, dn;  // gate/up interleaved and down in the grouped GEMM's layout (batches)
};

struct bb_stack {
  bb_ctx* ctx;
  std::vector<bb_layer_desc> layers;
  std::vector<float*> gains;
  float eps;
  int H;
  float* h = nullptr;
  float* h2 = nullptr;      // h alternates with h2 at boundaries that also route the next layer
  float* normed = nullptr;
  float* ffn = nullptr;
  float* logits = nullptr;  // the next MoE layer's router logits [T][32]
  int8_t* xq_q = nullptr;   // and the XQ records of its input
  float* xq_sx = nullptr;
  uint32_t* xq_pairs = nullptr;
  size_t cap_T = 0;
};

namespace {

void set_device(bb_ctx* c) { check_hip(hipSetDevice(c->device), "hipSetDevice"); }

// Set-up copies and clears go on the context's stream, which is then drained. (The context's
// stream does not wait for the null stream, so a plain hipMemcpy / hipMemset there may still
// be running when the stream's kernels read or write the same memory.)
void copy_to_dev(bb_ctx* c, void* dst, const void* src, size_t bytes, const char* what) {
  if (bytes == 0) return;
  check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream), what);
  check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}
void clear_dev(bb_ctx* c, void* dst, size_t bytes) {
  if (bytes == 0) return;
  check_hip(hipMemsetAsync(dst, 0, bytes, c->stream), "hipMemsetAsync");
  check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

hipEvent_t take_event(bb_ctx* c) {
  if (!c->event_pool.empty()) {
    hipEvent_t e = c->event_pool.back();
    c->event_pool.pop_back();
    return e;
  }
  hipEvent_t e;
  check_hip(hipEventCreate(&e), "hipEventCreate");
  return e;
}

// Launch wrapper: brackets the launch with events when profiling is on.
template <class F>
void launch(bb_ctx* c, int id, F&& f) {
  if (!c->profile) {
    check_hip(f(), bb::kernel_name(id));
    return;
  }
  // both events are recorded first (valid even if the launcher has nothing to launch); the
  // kernel's dispatch then re-stamps them with its exact start and end
  hipEvent_t a = take_event(c), b = take_event(c);
  check_hip(hipEventRecord(a, c->stream), "hipEventRecord");
  check_hip(hipEventRecord(b, c->stream), "hipEventRecord");
  bb::launch_events() = {a, b};
  const hipError_t rc = f();
  bb::launch_events() = {};
  check_hip(rc, bb::kernel_name(id));
  c->pending.push_back({id, a, b});
}

// The one-group route of T tokens for the grouped GEMM (counts, offsets, identity permutation),
// written into a carved buffer of T + 8 ints.
bb::RouteBufs one_group(bb_ctx* c, int32_t* grp, size_t T) {
  bb::RouteBufs rb{};
  rb.counts = grp;
  rb.offsets = grp + 2;
  rb.perm = grp + 8;
  launch(c, bb::K_DISPATCH, [&] { return bb::launch_one_group(c->stream, (int)T, rb); });
  return rb;
}

// y = W·x on the grouped GEMM for a packed W (p: plain 64-row tiles), x's Q8 rows in q.
void packed_project(bb_ctx* c, const bb::PackedW& p, size_t n_in, size_t n_out, size_t T, bb::Q8Bufs q,
                    const bb::RouteBufs& rb, float* y) {
  launch(c, bb::K_GEMM_DOWN, [&] {
    return bb::launch_gemm_down(c->stream, p.dt, p.w, p.stride, (int)T, (int)n_out, (int)n_in, 1, 1, rb,
                                bb::GemmX{q.q, q.scales}, y);
  });
}

void collect(bb_ctx* c) {
  if (c->pending.empty()) return;
  check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  for (auto& p : c->pending) {
    float ms = 0;
    check_hip(hipEventElapsedTime(&ms, p.a, p.b), "hipEventElapsedTime");
    c->kernel_ms[p.id] += ms;
    c->launches[p.id] += 1;
    c->event_pool.push_back(p.a);
    c->event_pool.push_back(p.b);
  }
  c->pending.clear();
}

uint8_t* ensure_ws(bb_ctx* c, size_t bytes) {
  if (bytes > c->ws_bytes) {
    check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (c->ws) (void)hipFree(c->ws);
    c->ws = nullptr;
    c->ws_bytes = 0;
    c->ws = static_cast<uint8_t*>(dev_alloc(bytes));
    c->ws_bytes = bytes;
    // selections read before any route wrote them must still name experts in range (cleared
    // on the context's stream, so that the clear lands before the stream's next kernels)
    check_hip(hipMemsetAsync(c->ws, 0, bytes, c->stream), "hipMemsetAsync");
  }
  return c->ws;
}

uint8_t* ensure_io(bb_ctx* c, size_t bytes) {
  if (bytes > c->io_bytes) {
    check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (c->io) (void)hipFree(c->io);
    c->io = nullptr;
    c->io_bytes = 0;
    c->io = static_cast<uint8_t*>(dev_alloc(bytes));
    c->io_bytes = bytes;
  }
  return c->io;
}

// Bump allocator over a byte region, 256-byte aligned slices.
struct Carve {
  uint8_t* base;
  size_t off = 0;
  template <class T>
  T* take(size_t n) {
    T* p = reinterpret_cast<T*>(base ? base + off : nullptr);
    off = round_up(off + n * sizeof(T), 256);
    return p;
  }
};

void need(bool ok, int code, const std::string& msg) {
  if (!ok) fail(code, msg);
}
// A nested call of this library's C ABI failed: rethrow with its code and message.
void check_code(int rc) {
  if (rc != BB_OK) fail(rc, std::string(g_err));
}
// string-literal form: builds no std::string unless the check fails
void need(bool ok, int code, const char* msg) {
  if (!ok) fail(code, msg);
}

void need_ctx(bb_ctx* c) { need(c != nullptr, BB_ERR_ARG, "null context"); }

void need_loc(int loc) { need(loc == BB_LOC_HOST || loc == BB_LOC_DEVICE, BB_ERR_ARG, "loc must be BB_LOC_HOST or BB_LOC_DEVICE"); }

void need_aligned(const void* p, const char* what) {
  if (p == nullptr) fail(BB_ERR_ARG, std::string(what) + " is null");
  if ((reinterpret_cast<uintptr_t>(p) & 15) != 0) fail(BB_ERR_ARG, std::string(what) + " must be 16-byte aligned");
}

size_t tensor_elems(const bb_tensor* t) {
  size_t n = 1;
  for (int i = 0; i < t->ndims; ++i) n *= t->dims[i];
  return n;
}

// ---- MoE forward on device pointers -----------------------------------------------------------

struct MoeWs {
  bb::XQBufs xq;
  bb::RouteBufs rb;
  float* act;
  float* slots;
  int8_t* aq;     // Q8 of act (batched path)
  float* aq_sx;
  uint16_t* aq_ms = nullptr;
};

// Workspace of one call: the context's (grown on demand) or a fixed region given by the caller
// (base, cap), which is never grown: a call that needs more fails with BB_ERR_RANGE.
struct WsRegion {
  uint8_t* base = nullptr;
  size_t cap = 0;
};

// Decode batches whose gate/up and down GEMMs both run as the kernels of at most 16 members
// (k_gateup16, k_down16): the Q8 act rows of expert e's member m go to row 16e + m (E·16 rows).
bool moe_act_pad(const bb_moe* m, size_t T) {
  const int n_ent = (int)(T * m->K);
  return bb::gateup16_applies((int)m->gu_dtype, (int)T, (int)m->H, (int)m->F, (int)m->E, (int)m->K,
                              !bb::gemm_reads_ms((int)m->dn_dtype, n_ent, (int)m->E)) &&
         bb::down16_applies((int)m->dn_dtype, (int)T, (int)m->H, (int)m->F, (int)m->E, (int)m->K);
}

MoeWs carve_moe(bb_ctx* c, const bb_moe* m, size_t T, bool batched, const WsRegion* fixed = nullptr) {
  const size_t H = m->H, F = m->F, E = m->E, K = m->K;
  for (int pass = 0; pass < 2; ++pass) {
    Carve cv{pass ? (fixed ? fixed->base : c->ws) : nullptr};
    MoeWs w{};
    w.xq.q = cv.take<int8_t>(T * H);
    w.xq.sx = cv.take<float>(T * H / 256);
    w.xq.pairs = batched ? nullptr : cv.take<uint32_t>(T * H / 256 * 12);
    w.xq.ms = batched && bb::gemm_reads_ms(m->gu_dtype, T * K, E) ? cv.take<uint16_t>(T * H / 256 * 16) : nullptr;
    w.rb.logits = cv.take<float>(T * E);
    w.rb.sel = cv.take<int32_t>(T * K);
    w.rb.wts = cv.take<float>(T * K);
    w.rb.counts = cv.take<int32_t>(E);
    w.rb.offsets = cv.take<int32_t>(E + 1);
    w.rb.perm = cv.take<int32_t>(T * K);
    w.rb.hit = cv.take<int32_t>(E + 1);
    w.rb.ties = cv.take<int32_t>(T);
    w.rb.margin = cv.take<float>(T);
    w.act = cv.take<float>(T * K * F);
    w.slots = cv.take<float>(T * K * H);
    if (batched) {
      const size_t aq_rows = moe_act_pad(m, T) ? std::max(T * K, 16 * E) : T * K;
      w.aq = cv.take<int8_t>(aq_rows * F);
      w.aq_sx = cv.take<float>(aq_rows * F / 256);
      w.aq_ms = bb::gemm_reads_ms(m->dn_dtype, T * K, E) ? cv.take<uint16_t>(T * K * F / 256 * 16) : nullptr;
    }
    if (pass == 0) {
      // the scratch area keeps the PAD bytes of tail slack every dev_alloc'd workspace has
      if (fixed)
        need(cv.off + PAD <= fixed->cap, BB_ERR_RANGE,
             "the call's workspace exceeds the allocation-free scratch area (BB_NOALLOC_SCRATCH_BYTES)");
      else
        ensure_ws(c, cv.off);
    } else {
      return w;
    }
  }
  return {};
}

// Router logits and XQ records of x computed before the call (by the stack's layer boundary).
struct PreRoute {
  const float* logits;
  bb::XQBufs xq;
};

// With combine false the caller combines: the slots and weights stay in the returned workspace.
// With pre set (a few tokens on the GEMV path only) the route's dots are already done.
// With fixed set the workspace is that region (nothing is allocated).
MoeWs moe_forward_dev(bb_ctx* c, bb_moe* m, const float* x, size_t T, float* out, bb_route_trace* tr,
                      bool combine = true, const PreRoute* pre = nullptr, const WsRegion* fixed = nullptr) {
  need(T >= 1, BB_ERR_ARG, "T must be >= 1");
  const size_t n_ent = T * (size_t)m->K;
  const bool batched = n_ent >= c->batched_min_entries;
  if (batched)
    need(n_ent <= (size_t)bb::PF_MAX_ENTRIES, BB_ERR_RANGE, "this path routes at most 32768 (token, slot) entries per call");
  else
    need(n_ent <= (size_t)bb::MAX_ENTRIES, BB_ERR_RANGE, "this path routes at most 1024 (token, slot) entries per call");
  MoeWs w = carve_moe(c, m, T, batched, fixed);
  const bool combine_in_down = !batched && combine && T == 1 && m->K <= 4 && m->H % 16 == 0 && m->F / 256 <= 8;
  if (batched) {
    // model.rs:286-371: route all tokens, group entries by expert, grouped GEMMs, combine
    launch(c, bb::K_ROUTE_LARGE, [&] {
      // tokens per routing block: each block reads the whole router once and then takes its
      // tokens one after the other (~1 µs each), so about one block per CU: ceil(T / CUs),
      // at most 16 (config 3 on 256 CUs: 2 tokens per block)
      const size_t n_cu = (size_t)c->n_cu;
      const int tpb = (int)std::max<size_t>(1, std::min<size_t>(16, (T + n_cu - 1) / n_cu));
      return bb::launch_route(c->stream, m->router_cm, m->bias_dev, x, (int)T, m->H, m->E, m->K, tpb, w.xq, w.rb);
    });
    // small batches: the GEMMs group the entries themselves; the dispatch kernel then only
    // fills the trace's counts, offsets and permutation
    if (bb::gemm_member_tiles((int)n_ent, m->E) > 1 || tr)
      launch(c, bb::K_DISPATCH, [&] { return bb::launch_dispatch(c->stream, (int)n_ent, m->E, w.rb); });
    // (decode batches: the gate/up kernel also writes the act rows' Q8 when it can)
    bool quantized = false;
    const bool act_pad = moe_act_pad(m, T);
    launch(c, bb::K_GEMM_GATEUP, [&] {
      return bb::launch_gemm_gateup(c->stream, m->gu_dtype, m->gu_packed, m->stride_gu, (int)T, m->H, m->F, m->E, m->K,
                                    w.rb, bb::GemmX{w.xq.q, w.xq.sx, w.xq.ms}, w.act, w.aq_ms ? nullptr : w.aq,
                                    w.aq_sx, &quantized, act_pad);
    });
    if (!quantized)
      launch(c, bb::K_QUANT, [&] {
        return bb::launch_quant_rows(c->stream, w.act, n_ent, m->F, w.aq, w.aq_sx, w.aq_ms);
      });
    launch(c, bb::K_GEMM_DOWN, [&] {
      return bb::launch_gemm_down(c->stream, m->dn_dtype, m->dn_packed, m->stride_dn, (int)T, m->H, m->F, m->E, m->K,
                                  w.rb, bb::GemmX{w.aq, w.aq_sx, w.aq_ms}, w.slots, act_pad);
    });
  } else {
    const int batch_mode = T > 1;
    const int max_hit = (int)std::min<size_t>((size_t)m->E, n_ent);
    // a few tokens: every gate/up block routes them itself (or only gates them, from logits
    // computed before the call)
    const bool route_in = T <= (size_t)bb::ROUTE_IN_GATEUP_MAX_T;
    need(!pre || route_in, BB_ERR_ARG, "routes computed before the call serve at most 4 tokens");
    if (!route_in)
      launch(c, bb::K_ROUTE, [&] {
        return bb::launch_route(c->stream, m->router_cm, m->bias_dev, x, (int)T, m->H, m->E, m->K, 1, w.xq, w.rb);
      });
    launch(c, bb::K_GATEUP, [&] {
      if (pre)
        return bb::launch_gate_gateup(c->stream, m->gu_dtype, m->gu_packed, m->stride_gu, (int)T, m->H, m->F, m->E,
                                      m->K, max_hit, batch_mode, tr != nullptr, w.rb, pre->logits, m->bias_dev,
                                      pre->xq, w.act);
      if (route_in)
        return bb::launch_route_gateup(c->stream, m->gu_dtype, m->gu_packed, m->stride_gu, (int)T, m->H, m->F, m->E,
                                       m->K, max_hit, batch_mode, tr != nullptr, w.rb, m->router_cm, m->bias_dev, x,
                                       w.act);
      return bb::launch_gateup(c->stream, m->gu_dtype, m->gu_packed, m->stride_gu, (int)T, m->H, m->F, m->E, m->K,
                               max_hit, batch_mode, tr != nullptr, w.rb, w.xq, w.act);
    });
    if (combine_in_down) {
      // one token: the down GEMV also combines (no slot rows)
      launch(c, bb::K_DOWN, [&] {
        return bb::launch_down_combine1(c->stream, m->dn_dtype, m->dn_packed, m->stride_dn, m->H, m->F, m->K, w.rb,
                                        w.act, out);
      });
    } else {
      launch(c, bb::K_DOWN, [&] {
        return bb::launch_down(c->stream, m->dn_dtype, m->dn_packed, m->stride_dn, (int)T, m->H, m->F, m->K, max_hit,
                               batch_mode, w.rb, w.act, w.slots);
      });
    }
  }
  if (combine && !combine_in_down)
    launch(c, bb::K_COMBINE, [&] { return bb::launch_combine(c->stream, w.slots, w.rb.wts, (int)T, m->H, m->K, out); });
  if (tr) {
    const size_t E = m->E, K = m->K;
    auto cp = [&](void* dst, const void* src, size_t bytes) {
      if (dst) check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream), "trace copy");
    };
    cp(tr->logits, w.rb.logits, T * E * 4);
    cp(tr->sel, w.rb.sel, T * K * 4);
    cp(tr->w, w.rb.wts, T * K * 4);
    cp(tr->counts, w.rb.counts, E * 4);
    cp(tr->offsets, w.rb.offsets, (E + 1) * 4);
    cp(tr->perm, w.rb.perm, T * K * 4);
    std::vector<int32_t> ties(T);
    cp(ties.data(), w.rb.ties, T * 4);
    cp(tr->margin, w.rb.margin, T * 4);
    check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (tr->ties) {
      int32_t tot = 0;
      for (int32_t v : ties) tot += v;
      *tr->ties = tot;
    }
  }
  return w;
}

// ---- dense FFN on device pointers (model.rs:459-469 / :262-278) --------------------------------
// xq_in (may be null): x's Q8, already computed (the decoder's fused residual + rmsnorm).
void dense_forward_dev(bb_ctx* c, bb_dense* d, const float* x, size_t T, float* out, const bb::Q8Bufs* xq_in = nullptr) {
  const size_t H = d->H, F = d->F;
  uint8_t* base = nullptr;
  for (int pass = 0; pass < 2; ++pass) {
    Carve cv{base};
    bb::Q8Bufs xq{cv.take<int8_t>(T * H), cv.take<float>(T * H / 256), cv.take<int32_t>(T * H / 32)};
    float* gate = cv.take<float>(T * F);
    float* up = cv.take<float>(T * F);
    bb::Q8Bufs aq{cv.take<int8_t>(T * F), cv.take<float>(T * F / 256), cv.take<int32_t>(T * F / 32)};
    int32_t* grp = cv.take<int32_t>(T + 8);
    if (pass == 0) {
      base = ensure_ws(c, cv.off);
      continue;
    }
    const int nz = T == 1;  // n_tokens == 1 takes matvec (-0.0-started sum), else matmul
    if (xq_in) xq = *xq_in;
    else launch(c, bb::K_QUANT, [&] { return bb::launch_quantize(c->stream, x, T, H, xq); });
    if (T >= bb::PROJ_GEMM_MIN_T && d->gu.w && d->dn.w) {
      // a batch: gate, up and swiglu, then down, as grouped GEMMs of one group (matmul's sums
      // from +0.0, the same per-(row, token) values as the row kernels)
      const bb::RouteBufs rb = one_group(c, grp, T);
      launch(c, bb::K_GEMM_GATEUP, [&] {
        return bb::launch_gemm_gateup(c->stream, d->gu.dt, d->gu.w, d->gu.stride, (int)T, (int)H, (int)F, 1, 1, rb,
                                      bb::GemmX{xq.q, xq.scales}, gate);
      });
      launch(c, bb::K_QUANT, [&] { return bb::launch_quant_rows(c->stream, gate, T, (int)F, aq.q, aq.scales); });
      packed_project(c, d->dn, F, H, T, aq, rb, out);
      continue;
    }
    const size_t gate_rb = (H / 256) * (d->gate->dtype == BB_Q4_K ? 144 : 210);
    if (d->gate->dtype == d->up->dtype && H / 256 <= 64) {
      // gate, up and swiglu in one pass over both matrices
      launch(c, bb::K_ROWS_Q8, [&] {
        return bb::launch_rows_q8_swiglu(c->stream, (int)d->gate->dtype, d->gate->dev, d->up->dev, gate_rb,
                                         (int)(H / 256), F, xq, H, T, gate, F, nz);
      });
    } else {
      launch(c, bb::K_ROWS_Q8, [&] {
        return bb::launch_rows_q8(c->stream, (int)d->gate->dtype, d->gate->dev, gate_rb, (int)(H / 256), F, xq, H, T,
                                  gate, F, nz);
      });
      launch(c, bb::K_ROWS_Q8, [&] {
        return bb::launch_rows_q8(c->stream, (int)d->up->dtype, d->up->dev,
                                  (H / 256) * (d->up->dtype == BB_Q4_K ? 144 : 210), (int)(H / 256), F, xq, H, T, up,
                                  F, nz);
      });
      launch(c, bb::K_ELEMWISE,
             [&] { return bb::launch_elementwise(c->stream, bb::EW_SWIGLU, gate, gate, up, 0.f, T * F); });
    }
    launch(c, bb::K_QUANT, [&] { return bb::launch_quantize(c->stream, gate, T, F, aq); });
    launch(c, bb::K_ROWS_Q8, [&] {
      return bb::launch_rows_q8(c->stream, (int)d->down->dtype, d->down->dev,
                                (F / 256) * (d->down->dtype == BB_Q4_K ? 144 : 210), (int)(F / 256), H, aq, F, T, out,
                                H, nz);
    });
  }
}

// Runs `body(ptr_map)` with host arrays staged through the context's io buffer.
struct Io {
  const void* host;
  size_t bytes;
  bool in, out;
};

template <class F>
void with_io(bb_ctx* c, int loc, std::vector<Io> ios, F&& body) {
  std::vector<void*> dev(ios.size());
  if (loc == BB_LOC_DEVICE) {
    for (size_t i = 0; i < ios.size(); ++i) {
      if (ios[i].bytes) need_aligned(ios[i].host, "device pointer");
      dev[i] = const_cast<void*>(ios[i].host);
    }
    body(dev);
    return;
  }
  size_t total = 0;
  for (auto& io : ios) total = round_up(total + io.bytes, 256);
  uint8_t* base = ensure_io(c, total + 256);
  size_t off = 0;
  for (size_t i = 0; i < ios.size(); ++i) {
    if (ios[i].bytes) need(ios[i].host != nullptr, BB_ERR_ARG, "null host pointer");
    dev[i] = base + off;
    if (ios[i].in && ios[i].bytes)
      check_hip(hipMemcpyAsync(dev[i], ios[i].host, ios[i].bytes, hipMemcpyHostToDevice, c->stream), "H2D copy");
    off = round_up(off + ios[i].bytes, 256);
  }
  body(dev);
  for (size_t i = 0; i < ios.size(); ++i)
    if (ios[i].out && ios[i].bytes)
      check_hip(hipMemcpyAsync(const_cast<void*>(ios[i].host), dev[i], ios[i].bytes, hipMemcpyDeviceToHost, c->stream),
                "D2H copy");
  check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

void check_weight_range(const bb_tensor* w, uint32_t dtype, size_t byte_off, size_t n_in, size_t n_out,
                        size_t& row_bytes) {
  need(w != nullptr, BB_ERR_ARG, "null weight tensor");
  size_t be, bb_;
  need(block_of(dtype, be, bb_), BB_ERR_DTYPE, "unsupported weight dtype " + std::to_string(dtype));
  need(dtype == w->dtype, BB_ERR_DTYPE, "dtype does not match the uploaded tensor's");
  need(n_in % be == 0, BB_ERR_SHAPE, "n_in (" + std::to_string(n_in) + ") not a multiple of block (" + std::to_string(be) + ")");
  row_bytes = (n_in / be) * bb_;
  need(byte_off + row_bytes * n_out <= w->nbytes, BB_ERR_SHAPE, "weight slice exceeds the tensor");
  if (dtype == BB_Q4_K) need(byte_off % 16 == 0, BB_ERR_ARG, "Q4_K slices must start 16-byte aligned");
  if (dtype == BB_Q6_K) need(byte_off % 2 == 0, BB_ERR_ARG, "Q6_K slices must start 2-byte aligned");
  if (dtype == BB_F32) need(byte_off % 4 == 0, BB_ERR_ARG, "F32 slices must start 4-byte aligned");
  if (dtype == BB_F16) need(byte_off % 2 == 0, BB_ERR_ARG, "F16 slices must start 2-byte aligned");
}

// matvec / matmul on device pointers.
void matmul_dev(bb_ctx* c, uint32_t dtype, const bb_tensor* w, size_t byte_off, size_t n_in, size_t n_out,
                const float* x, size_t nt, float* y) {
  size_t row_bytes;
  check_weight_range(w, dtype, byte_off, n_in, n_out, row_bytes);
  const uint8_t* wp = w->dev + byte_off;
  if (dtype == BB_Q4_K || dtype == BB_Q6_K) {
    Carve cv{nullptr};
    cv.take<int8_t>(nt * n_in);
    cv.take<float>(nt * n_in / 256);
    cv.take<int32_t>(nt * n_in / 32);
    uint8_t* base = ensure_ws(c, cv.off);
    Carve cv2{base};
    bb::Q8Bufs q{cv2.take<int8_t>(nt * n_in), cv2.take<float>(nt * n_in / 256), cv2.take<int32_t>(nt * n_in / 32)};
    launch(c, bb::K_QUANT, [&] { return bb::launch_quantize(c->stream, x, nt, n_in, q); });
    launch(c, bb::K_ROWS_Q8, [&] {
      return bb::launch_rows_q8(c->stream, (int)dtype, wp, row_bytes, (int)(n_in / 256), n_out, q, n_in, nt, y, n_out,
                                nt == 1);
    });
  } else {
    launch(c, bb::K_ROWS_F32, [&] { return bb::launch_rows_f32(c->stream, (int)dtype, wp, n_in, n_out, x, nt, y); });
  }
}

// ---- decoder-layer operators (bb_ops.hip) ----------------------------------------------------
// Q8 buffers of one projection input (T rows of n_in), carved like the other workspaces.
bb::Q8Bufs carve_q8(Carve& cv, size_t T, size_t n_in) {
  return {cv.take<int8_t>(T * n_in), cv.take<float>(T * n_in / 256), cv.take<int32_t>(T * n_in / 32)};
}

// y = W·x for T token-major rows as the reference's operators call it: matvec1 for one token
// (model.rs:557-560), matmul1 for a batch (:372-375); both are the row kernels (the one-token
// form sums from -0.0 as matvec does). q: Q8 buffers for x when W is Q4_K / Q6_K.
// With a packed form and a one-group route (rb non-null: batches of PROJ_GEMM_MIN_T tokens and
// more) the batch runs on the grouped GEMM instead.
// q_ready: q already holds x's Q8 (quants, scales and sums), so no quantisation is launched.
void project_dev(bb_ctx* c, const bb_tensor* w, const bb::PackedW& pk, const bb::RouteBufs* rb, size_t n_in,
                 size_t n_out, const float* x, size_t T, float* y, bb::Q8Bufs q, bool q_ready = false) {
  size_t row_bytes;
  check_weight_range(w, w->dtype, 0, n_in, n_out, row_bytes);
  if (pk.w && rb) {
    if (!q_ready)
      launch(c, bb::K_QUANT, [&] { return bb::launch_quant_rows(c->stream, x, T, (int)n_in, q.q, q.scales); });
    packed_project(c, pk, n_in, n_out, T, q, *rb, y);
    return;
  }
  if (w->dtype == BB_Q4_K || w->dtype == BB_Q6_K) {
    if (!q_ready) launch(c, bb::K_QUANT, [&] { return bb::launch_quantize(c->stream, x, T, n_in, q); });
    launch(c, bb::K_ROWS_Q8, [&] {
      return bb::launch_rows_q8(c->stream, (int)w->dtype, w->dev, row_bytes, (int)(n_in / 256), n_out, q, n_in, T, y,
                                n_out, T == 1);
    });
  } else {
    launch(c, bb::K_ROWS_F32, [&] { return bb::launch_rows_f32(c->stream, (int)w->dtype, w->dev, n_in, n_out, x, T, y); });
  }
}

void need_proj(const bb_tensor* t, uint64_t n_in, uint64_t n_out, const char* what) {
  need(t != nullptr, BB_ERR_ARG, std::string(what) + " is null");
  need(t->ndims == 2 && t->dims[0] == n_in && t->dims[1] == n_out, BB_ERR_SHAPE,
       std::string(what) + " must be [" + std::to_string(n_in) + ", " + std::to_string(n_out) + "]");
  need(t->dtype == BB_Q4_K || t->dtype == BB_Q6_K || t->dtype == BB_F32 || t->dtype == BB_F16, BB_ERR_DTYPE,
       std::string(what) + ": dtype must be F32, F16, Q4_K or Q6_K");
  if (t->dtype == BB_Q4_K || t->dtype == BB_Q6_K) need(n_in % 256 == 0, BB_ERR_SHAPE, "n_in must be a multiple of 256");
}

float* upload_f32(bb_ctx* c, const float* host, size_t n) {
  float* d = static_cast<float*>(dev_alloc(n * 4));
  try {
    copy_to_dev(c, d, host, n * 4, "host array upload");
  } catch (...) {
    (void)hipFree(d);
    throw;
  }
  return d;
}

// The grouped GEMM's packed form of a projection (one expert): plain 64-row tiles of w, or gate
// and up interleaved (up != null). Empty (w null) when the dtype or shape has no packed form.
bb::PackedW pack_weights(bb_ctx* c, const bb_tensor* w, const bb_tensor* up, size_t n_in, size_t n_out) {
  bb::PackedW p;
  const uint32_t dt = w->dtype;
  if (dt != BB_Q4_K && dt != BB_Q6_K) return p;
  if (up && up->dtype != dt) return p;
  if (n_in % 256 != 0 || n_out % (up ? 64 : 128) != 0) return p;
  const size_t nb = n_in / 256, row_bytes = nb * (dt == BB_Q4_K ? 144 : 210);
  p.dt = (int)dt;
  p.stride = (up ? n_out / 32 : n_out / 64) * nb * bb::pack_tile_block_bytes((int)dt);
  p.w = static_cast<uint8_t*>(dev_alloc(p.stride));
  const hipError_t e = bb::launch_pack_rows(c->stream, (int)dt, w->dev, up ? up->dev : nullptr, n_out * row_bytes,
                                            up ? n_out * row_bytes : 0, (int)n_out, (int)nb, 1, p.w);
  const hipError_t e2 = e == hipSuccess ? hipStreamSynchronize(c->stream) : e;
  if (e2 != hipSuccess) {
    (void)hipFree(p.w);
    check_hip(e2, "weight packing");
  }
  return p;
}

void free_packed(bb::PackedW& p) {
  if (p.w) (void)hipFree(p.w);
  p = bb::PackedW();
}

// (cos, sin) of RoPE pair i at `pos` as rope.rs:17-30 computes them: theta from (float)pos,
// multiplied by powf(base, -2/d) after each pair; libm's sinf / cosf (what f32::sin_cos calls).
void rope_rows(std::vector<float2>& out, size_t pos0, size_t n_pos, size_t hd, float freq_base) {
  const size_t half = hd / 2;
  const float theta_scale = std::pow(freq_base, -2.0f / float(hd));
  out.resize(n_pos * half);
  for (size_t p = 0; p < n_pos; ++p) {
    float theta = float(pos0 + p);
    for (size_t i = 0; i < half; ++i) {
      out[p * half + i] = make_float2(std::cos(theta), std::sin(theta));
      theta *= theta_scale;
    }
  }
}

// Model::logits_from_hidden (model.rs:380-388) on device pointers: rmsnorm(h, gain, eps), then
// the token_embd matvec (hidden -> vocab).
void logits_dev(bb_ctx* c, const bb_tensor* tok_embd, const float* gain, float eps, const float* h, float* logits) {
  const size_t H = tok_embd->dims[0], V = tok_embd->dims[1];
  const uint32_t dt = tok_embd->dtype;
  if ((dt == BB_Q4_K || dt == BB_Q6_K) && H % 256 == 0 && H <= (size_t)bb::GU_H_MAX) {
    // one launch for the rmsnorm and the Q8 of the normed row, then the rows
    size_t row_bytes;
    check_weight_range(tok_embd, dt, 0, H, V, row_bytes);
    Carve cv{nullptr};
    cv.take<int8_t>(H);
    cv.take<float>(H / 256);
    cv.take<int32_t>(H / 32);
    Carve cv2{ensure_ws(c, cv.off)};
    bb::Q8Bufs q{cv2.take<int8_t>(H), cv2.take<float>(H / 256), cv2.take<int32_t>(H / 32)};
    launch(c, bb::K_RMSNORM, [&] { return bb::launch_rmsnorm_q8(c->stream, h, gain, eps, H, 1, nullptr, q); });
    launch(c, bb::K_ROWS_Q8, [&] {
      return bb::launch_rows_q8(c->stream, (int)dt, tok_embd->dev, row_bytes, (int)(H / 256), V, q, H, 1, logits, V, 1);
    });
    return;
  }
  // normed lives past the Q8 records matmul_dev carves from the workspace's start
  Carve cv{nullptr};
  cv.take<int8_t>(H);
  cv.take<float>(H / 256);
  cv.take<int32_t>(H / 32);
  const size_t q8_bytes = cv.off;
  cv.take<float>(H);
  float* normed = reinterpret_cast<float*>(ensure_ws(c, cv.off) + q8_bytes);
  launch(c, bb::K_RMSNORM, [&] { return bb::launch_rmsnorm(c->stream, h, gain, eps, H, 1, normed); });
  matmul_dev(c, tok_embd->dtype, tok_embd, 0, H, V, normed, 1, logits);
}

}  // namespace

struct bb_conv_op {
  bb_ctx* ctx;
  const bb_tensor* in_proj;
  const bb_tensor* out_proj;
  float* conv_w;  // device, [hidden][l_cache]
  int H, L;
  bb::PackedW in_p, out_p;  // the projections in the grouped GEMM's layout (batches)
};

struct bb_kv_cache {
  bb_ctx* ctx;
  float* k;
  float* v;
  size_t kv_dim, cap, n;
};

struct bb_attn_op {
  bb_ctx* ctx;
  const bb_tensor *q, *k, *v, *o;
  bb::PackedW q_p, k_p, v_p, o_p;  // the projections in the grouped GEMM's layout (batches)
  float *q_norm, *k_norm;  // device, [head_dim]
  int H, NH, NKV, HD;
  float eps, freq_base, scale;
  float2* rope = nullptr;  // device (cos, sin) rows [rope_rows][head_dim/2] for positions 0..
  size_t rope_rows = 0;
};

// The decoder's weights (Model, model.rs:25-31): embedding, layers of (attn_norm, conv or
// attention operator, ffn_norm, dense or MoE FFN), final norm and logits. Immutable once built;
// the decode-time state lives in bb_cache. The buffers below are per-call scratch of the
// model's context (its calls are ordered on that context's stream).
struct bb_model {
  bb_ctx* ctx;
  const bb_tensor* tok_embd;
  float* final_norm;  // device
  float eps;
  int H;
  size_t vocab, row_bytes;
  struct Layer {
    float* attn_norm;  // device
    float* ffn_norm;
    bb_conv_op* conv;
    bb_attn_op* attn;
    bb_moe* moe;
    bb_dense* dense;
  };
  std::vector<Layer> layers;
  float *h = nullptr, *normed = nullptr, *tmp = nullptr;
  bb::Q8Bufs nq{};          // Q8 of normed, written with it for the conv / attention / dense layers
  // a boundary before an MoE layer of a few tokens also takes its router logits and XQ records
  // (the residual then goes to h2, which becomes h)
  float *h2 = nullptr, *logits = nullptr;
  bb::XQBufs xq{};
  uint32_t* tok = nullptr;  // token ids of the current call
  size_t cap_T = 0, tok_cap = 0;
  bb::ModelOwned owned;  // set by bb_model_load
};

// Decode-time state of one conversation (Cache, cache.rs:10-19) for the layers of one model:
// a conv state per conv layer, a device KV cache per attention layer (grown on demand, as the
// reference's Vec histories grow), and the next token's position.
struct bb_cache {
  bb_ctx* ctx;
  const bb_model* model;
  std::vector<float*> conv;       // per layer: [(L-1)][H] for conv layers, else null
  std::vector<bb_kv_cache*> kv;   // per layer: attention layers, else null
  size_t pos = 0;
};

void bb::free_owned(bb::ModelOwned& o) {
  for (bb_conv_op* p : o.conv) (void)bb_conv_op_destroy(p);
  for (bb_attn_op* p : o.attn) (void)bb_attn_op_destroy(p);
  for (bb_moe* p : o.moe) (void)bb_moe_destroy(p);
  for (bb_dense* p : o.dense) (void)bb_dense_destroy(p);
  for (bb_tensor* p : o.tensors) (void)bb_tensor_free(p);
  o = bb::ModelOwned();
}

void bb::model_adopt(bb_model* m, bb::ModelOwned&& o) { m->owned = std::move(o); }

namespace {

// model.rs:399-427 (T == 1) and :190-216 (T > 1) on device pointers; state [(L-1)][H] is updated.
void conv_forward_dev(bb_ctx* c, bb_conv_op* op, float* state, const float* x, size_t T, float* out,
                      const bb::Q8Bufs* xq_in = nullptr) {
  const size_t H = op->H;
  uint8_t* base = nullptr;
  for (int pass = 0; pass < 2; ++pass) {
    Carve cv{base};
    bb::Q8Bufs xq = carve_q8(cv, T, H);
    float* bcx = cv.take<float>(T * 3 * H);
    float* y = cv.take<float>(T * H);
    bb::Q8Bufs yq = carve_q8(cv, T, H);
    int32_t* grp = cv.take<int32_t>(T + 8);
    if (pass == 0) {
      base = ensure_ws(c, cv.off);
      continue;
    }
    bb::RouteBufs rb{};
    const bool gemm = T >= bb::PROJ_GEMM_MIN_T && (op->in_p.w || op->out_p.w);
    if (gemm) rb = one_group(c, grp, T);
    project_dev(c, op->in_proj, op->in_p, gemm ? &rb : nullptr, H, 3 * H, x, T, bcx, xq_in ? *xq_in : xq,
                xq_in != nullptr);
    if (T == 1 && H % 256 == 0 && (op->out_proj->dtype == BB_Q4_K || op->out_proj->dtype == BB_Q6_K)) {
      // one token: conv, state update and y's Q8 in one launch
      launch(c, bb::K_CONV, [&] { return bb::launch_conv1_q8(c->stream, bcx, state, op->conv_w, (int)H, op->L, y, yq); });
      project_dev(c, op->out_proj, op->out_p, nullptr, H, H, y, T, out, yq, true);
      continue;
    }
    launch(c, bb::K_CONV, [&] { return bb::launch_conv(c->stream, true, bcx, state, op->conv_w, (int)H, op->L, (int)T, y); });
    launch(c, bb::K_CONV_STATE, [&] { return bb::launch_conv_state(c->stream, true, bcx, state, (int)H, op->L, (int)T); });
    project_dev(c, op->out_proj, op->out_p, gemm ? &rb : nullptr, H, H, y, T, out, yq);
  }
}

// Grows the op's RoPE table to at least `rows` positions (recomputed on the host, uploaded once).
void ensure_rope(bb_ctx* c, bb_attn_op* op, size_t rows) {
  if (rows <= op->rope_rows) return;
  const size_t n = std::max<size_t>({rows, 2 * op->rope_rows, 4096});
  std::vector<float2> tab;
  rope_rows(tab, 0, n, op->HD, op->freq_base);
  auto* d = static_cast<float2*>(dev_alloc(tab.size() * sizeof(float2)));
  try {
    copy_to_dev(c, d, tab.data(), tab.size() * sizeof(float2), "RoPE table upload");  // (drains the stream)
  } catch (...) {
    (void)hipFree(d);
    throw;
  }
  if (op->rope) (void)hipFree(op->rope);
  op->rope = d;
  op->rope_rows = n;
}

// model.rs:430-456 (T == 1) and :222-259 (T > 1) on device pointers: the T new keys / values
// are projected straight into the cache rows n .. n+T-1.
void attn_forward_dev(bb_ctx* c, bb_attn_op* op, bb_kv_cache* kv, size_t pos0, const float* x, size_t T, float* out,
                      const bb::Q8Bufs* xq_in = nullptr) {
  const size_t H = op->H, NH = op->NH, NKV = op->NKV, HD = op->HD, KV = NKV * HD, QD = NH * HD;
  const size_t n0 = kv->n;
  ensure_rope(c, op, pos0 + T);
  uint8_t* base = nullptr;
  for (int pass = 0; pass < 2; ++pass) {
    Carve cv{base};
    bb::Q8Bufs xq = carve_q8(cv, T, H);
    float* q = cv.take<float>(T * QD);
    float* scores = cv.take<float>(T * NH * (n0 + T) + 4);  // (+ slack: launch_attn_pv reads one float past the rows)
    float* attn = cv.take<float>(T * QD);
    bb::Q8Bufs aq = carve_q8(cv, T, QD);
    int32_t* grp = cv.take<int32_t>(T + 8);
    if (pass == 0) {
      base = ensure_ws(c, cv.off);
      continue;
    }
    float* kn = kv->k + n0 * KV;
    float* vn = kv->v + n0 * KV;
    bb::RouteBufs rb{};
    const bool gemm = T >= bb::PROJ_GEMM_MIN_T && (op->q_p.w || op->k_p.w || op->v_p.w || op->o_p.w);
    if (gemm) rb = one_group(c, grp, T);
    const bb::RouteBufs* rbp = gemm ? &rb : nullptr;
    // x's Q8 (quants, scales and sums: both the row kernels and the GEMMs can read it) once for
    // the three projections, or as given
    const bb::Q8Bufs xqv = xq_in ? *xq_in : xq;
    if (!xq_in && (op->q->dtype == BB_Q4_K || op->q->dtype == BB_Q6_K || op->k->dtype == BB_Q4_K ||
                   op->k->dtype == BB_Q6_K || op->v->dtype == BB_Q4_K || op->v->dtype == BB_Q6_K))
      launch(c, bb::K_QUANT, [&] { return bb::launch_quantize(c->stream, x, T, H, xq); });
    project_dev(c, op->q, op->q_p, rbp, H, QD, x, T, q, xqv, true);
    project_dev(c, op->k, op->k_p, rbp, H, KV, x, T, kn, xqv, true);
    project_dev(c, op->v, op->v_p, rbp, H, KV, x, T, vn, xqv, true);
    const float2* rope = op->rope + pos0 * (HD / 2);
    launch(c, bb::K_NORM_ROPE, [&] {
      return bb::launch_norm_rope(c->stream, q, (int)T, (int)NH, (int)HD, op->q_norm, op->eps, rope, kn, (int)NKV,
                                  op->k_norm);
    });
    launch(c, bb::K_ATTN_SCORES, [&] {
      return bb::launch_attn_scores(c->stream, q, kv->k, (int)n0, (int)T, (int)NH, (int)NKV, (int)HD, op->scale, scores);
    });
    launch(c, bb::K_ATTN_PV, [&] {
      return bb::launch_attn_pv(c->stream, scores, kv->v, (int)n0, (int)T, (int)NH, (int)NKV, (int)HD, attn);
    });
    project_dev(c, op->o, op->o_p, rbp, QD, H, attn, T, out, aq);
  }
  kv->n = n0 + T;
}

}  // namespace

extern "C" {

const char* bb_last_error(void) { return g_err.c_str(); }
const char* bb_version(void) { return "bebelm_moe 0.1.0 (gfx950)"; }

int bb_ctx_create(int device, bb_ctx** out) {
  return guard([&] {
    need(out != nullptr, BB_ERR_ARG, "out is null");
    int n = 0;
    check_hip(hipGetDeviceCount(&n), "hipGetDeviceCount");
    need(device >= 0 && device < n, BB_ERR_ARG, "no such device " + std::to_string(device));
    auto* c = new bb_ctx();
    c->device = device;
    try {
      set_device(c);
      check_hip(hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking), "hipStreamCreate");
      c->stream = c->own;
      int n_cu = 0;
      check_hip(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, device), "hipDeviceGetAttribute");
      c->n_cu = n_cu > 0 ? n_cu : 256;
      if (device < SCRATCH_MAX_DEVICES) {
        // the device's copy of the allocation-free scratch area: its address, and cleared once
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        if (!g_scratch[device]) {
          void* p = nullptr;
          check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
          check_hip(hipMemsetAsync(p, 0, BB_NOALLOC_SCRATCH_BYTES, c->own), "scratch clear");
          check_hip(hipStreamSynchronize(c->own), "hipStreamSynchronize");
          g_scratch[device] = static_cast<uint8_t*>(p);
        }
      }
      check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
    } catch (...) {
      if (c->own) (void)hipStreamDestroy(c->own);
      delete c;
      throw;
    }
    *out = c;
  });
}

int bb_ctx_destroy(bb_ctx* c) {
  return guard([&] {
    if (!c) return;
    set_device(c);
    (void)hipStreamSynchronize(c->stream);
    for (auto& p : c->pending) {
      (void)hipEventDestroy(p.a);
      (void)hipEventDestroy(p.b);
    }
    for (auto e : c->event_pool) (void)hipEventDestroy(e);
    if (c->ws) (void)hipFree(c->ws);
    if (c->io) (void)hipFree(c->io);
    if (c->own) (void)hipStreamDestroy(c->own);
    delete c;
  });
}

int bb_ctx_set_stream(bb_ctx* c, void* s) {
  return guard([&] {
    need_ctx(c);
    c->stream = s ? static_cast<hipStream_t>(s) : c->own;
  });
}

int bb_ctx_get_stream(bb_ctx* c, void** s) {
  return guard([&] {
    need_ctx(c);
    need(s != nullptr, BB_ERR_ARG, "out is null");
    *s = c->stream;
  });
}

int bb_ctx_synchronize(bb_ctx* c) {
  return guard([&] {
    need_ctx(c);
    set_device(c);
    check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  });
}

int bb_ctx_profile(bb_ctx* c, int enable) {
  return guard([&] {
    need_ctx(c);
    collect(c);
    c->profile = enable != 0;
  });
}

int bb_kernel_count(void) { return bb::K_COUNT; }

int bb_ctx_kernel_stats(bb_ctx* c, int idx, const char** name, double* total_ms, int64_t* launches) {
  return guard([&] {
    need_ctx(c);
    need(idx >= 0 && idx < bb::K_COUNT, BB_ERR_ARG, "kernel index out of range");
    collect(c);
    if (name) *name = bb::kernel_name(idx);
    if (total_ms) *total_ms = c->kernel_ms[idx];
    if (launches) *launches = c->launches[idx];
  });
}

int bb_ctx_reset_stats(bb_ctx* c) {
  return guard([&] {
    need_ctx(c);
    collect(c);
    for (int i = 0; i < bb::K_COUNT; ++i) {
      c->kernel_ms[i] = 0;
      c->launches[i] = 0;
    }
  });
}

int bb_ctx_set_batched_min_entries(bb_ctx* c, size_t min_entries) {
  return guard([&] {
    need_ctx(c);
    c->batched_min_entries = min_entries;
  });
}

int bb_tensor_upload(bb_ctx* c, uint32_t dtype, const void* bytes, size_t nbytes, const uint64_t* dims, int ndims,
                     bb_tensor** out) {
  return guard([&] {
    need_ctx(c);
    need(out != nullptr && bytes != nullptr && dims != nullptr, BB_ERR_ARG, "null argument");
    need(ndims >= 1 && ndims <= 4, BB_ERR_ARG, "ndims must be 1..4");
    size_t be, bb_;
    need(block_of(dtype, be, bb_), BB_ERR_DTYPE, "unsupported dtype " + std::to_string(dtype));
    size_t n = 1;
    for (int i = 0; i < ndims; ++i) n *= dims[i];
    need(n % be == 0, BB_ERR_SHAPE, "element count is not a whole number of blocks");
    need((n / be) * bb_ == nbytes, BB_ERR_SHAPE,
         "nbytes " + std::to_string(nbytes) + " != byte_size " + std::to_string((n / be) * bb_));
    set_device(c);
    auto* t = new bb_tensor();
    t->ctx = c;
    t->dtype = dtype;
    t->ndims = ndims;
    for (int i = 0; i < 4; ++i) t->dims[i] = i < ndims ? dims[i] : 1;
    t->nbytes = nbytes;
    try {
      t->dev = static_cast<uint8_t*>(dev_alloc(nbytes));
      check_hip(hipMemsetAsync(t->dev + nbytes, 0, round_up(nbytes, 256) + PAD - nbytes, c->stream), "pad clear");
      copy_to_dev(c, t->dev, bytes, nbytes, "upload");
    } catch (...) {
      if (t->dev) (void)hipFree(t->dev);
      delete t;
      throw;
    }
    *out = t;
  });
}

int bb_tensor_free(bb_tensor* t) {
  return guard([&] {
    if (!t) return;
    set_device(t->ctx);
    (void)hipStreamSynchronize(t->ctx->stream);
    (void)hipFree(t->dev);
    delete t;
  });
}

int bb_tensor_device_ptr(const bb_tensor* t, void** dev) {
  return guard([&] {
    need(t != nullptr && dev != nullptr, BB_ERR_ARG, "null argument");
    *dev = t->dev;
  });
}

int bb_quantize_q8(bb_ctx* c, const float* x, size_t n, int8_t* q, float* scales, int32_t* sums, int loc) {
  return guard([&] {
    need_ctx(c);
    need_loc(loc);
    need(n % 256 == 0, BB_ERR_SHAPE, "quantize_q8: n must be a multiple of 256");
    set_device(c);
    with_io(c, loc, {{x, n * 4, true, false}, {q, n, false, true}, {scales, n / 256 * 4, false, true}, {sums, n / 32 * 4, false, true}},
            [&](std::vector<void*>& d) {
              bb::Q8Bufs qb{static_cast<int8_t*>(d[1]), static_cast<float*>(d[2]), static_cast<int32_t*>(d[3])};
              launch(c, bb::K_QUANT, [&] { return bb::launch_quantize(c->stream, static_cast<const float*>(d[0]), 1, n, qb); });
            });
  });
}

int bb_matvec(bb_ctx* c, uint32_t dtype, const bb_tensor* w, size_t byte_off, size_t n_in, size_t n_out,
              const float* x, float* y, int loc) {
  return bb_matmul(c, dtype, w, byte_off, n_in, n_out, x, 1, y, loc);
}

int bb_matmul(bb_ctx* c, uint32_t dtype, const bb_tensor* w, size_t byte_off, size_t n_in, size_t n_out,
              const float* x, size_t n_tokens, float* y, int loc) {
  return guard([&] {
    need_ctx(c);
    need_loc(loc);
    need(n_tokens >= 1, BB_ERR_ARG, "n_tokens must be >= 1");
    size_t rb;
    check_weight_range(w, dtype, byte_off, n_in, n_out, rb);
    set_device(c);
    with_io(c, loc, {{x, n_in * n_tokens * 4, true, false}, {y, n_out * n_tokens * 4, false, true}},
            [&](std::vector<void*>& d) {
              matmul_dev(c, dtype, w, byte_off, n_in, n_out, static_cast<const float*>(d[0]), n_tokens,
                         static_cast<float*>(d[1]));
            });
  });
}

int bb_matvec_fused_batch(bb_ctx* c, const bb_fused_job* jobs, size_t n_jobs, float* out, int loc) {
  return guard([&] {
    need_ctx(c);
    need_loc(loc);
    need(jobs != nullptr || n_jobs == 0, BB_ERR_ARG, "jobs is null");
    size_t total = 0;
    std::vector<size_t> rbytes(n_jobs);
    for (size_t j = 0; j < n_jobs; ++j) {
      // (F32 / F16 jobs have no fused path: fused_row_dot panics on them, matmul.rs:783)
      need(jobs[j].dtype == BB_Q4_K || jobs[j].dtype == BB_Q6_K, BB_ERR_DTYPE,
           "matvec_fused_batch: jobs must be Q4_K or Q6_K");
      need(jobs[j].qx_q != nullptr || jobs[j].x != nullptr, BB_ERR_ARG, "matvec_fused_batch: a job has neither qx nor x");
      check_weight_range(jobs[j].w, jobs[j].dtype, jobs[j].byte_off, jobs[j].n_in, jobs[j].n_out, rbytes[j]);
      total += jobs[j].n_out;
    }
    set_device(c);
    std::vector<Io> ios;
    std::vector<size_t> first(n_jobs);  // the job's first entry in ios
    for (size_t j = 0; j < n_jobs; ++j) {
      first[j] = ios.size();
      if (jobs[j].qx_q) {
        ios.push_back({jobs[j].qx_q, jobs[j].n_in, true, false});
        ios.push_back({jobs[j].qx_scales, jobs[j].n_in / 256 * 4, true, false});
        ios.push_back({jobs[j].qx_sums, jobs[j].n_in / 32 * 4, true, false});
      } else {
        ios.push_back({jobs[j].x, jobs[j].n_in * 4, true, false});
      }
    }
    ios.push_back({out, total * 4, false, true});
    with_io(c, loc, ios, [&](std::vector<void*>& d) {
      float* o = static_cast<float*>(d.back());
      size_t start = 0;
      for (size_t j = 0; j < n_jobs; ++j) {
        const bb_fused_job& jb = jobs[j];
        const size_t f = first[j];
        if (jb.qx_q) {
          bb::Q8Bufs q{static_cast<int8_t*>(d[f]), static_cast<float*>(d[f + 1]), static_cast<int32_t*>(d[f + 2])};
          launch(c, bb::K_ROWS_Q8, [&] {
            return bb::launch_rows_q8(c->stream, (int)jb.dtype, jb.w->dev + jb.byte_off, rbytes[j],
                                      (int)(jb.n_in / 256), jb.n_out, q, jb.n_in, 1, o + start, jb.n_out, 1);
          });
        } else {
          launch(c, bb::K_ROWS_F32, [&] {
            return bb::launch_fused_rows_f32(c->stream, (int)jb.dtype, jb.w->dev + jb.byte_off, rbytes[j],
                                             (int)(jb.n_in / 256), jb.n_out, static_cast<const float*>(d[f]),
                                             o + start);
          });
        }
        start += jb.n_out;
      }
    });
  });
}

static int elementwise(bb_ctx* c, int op, float* out, const float* a, const float* b, float s, size_t n, int loc) {
  return guard([&] {
    need_ctx(c);
    need_loc(loc);
    set_device(c);
    std::vector<Io> ios{{out, n * 4, op != bb::EW_SWIGLU, true}, {a, n * 4, true, false}};
    if (op == bb::EW_SWIGLU) ios.push_back({b, n * 4, true, false});
    with_io(c, loc, ios, [&](std::vector<void*>& d) {
      launch(c, bb::K_ELEMWISE, [&] {
        return bb::launch_elementwise(c->stream, op, static_cast<float*>(d[0]), static_cast<const float*>(d[1]),
                                      op == bb::EW_SWIGLU ? static_cast<const float*>(d[2]) : nullptr, s, n);
      });
    });
  });
}

int bb_swiglu(bb_ctx* c, const float* gate, const float* up, float* out, size_t n, int loc) {
  return elementwise(c, bb::EW_SWIGLU, out, gate, up, 0.f, n, loc);
}
int bb_sigmoid_slice(bb_ctx* c, float* x, size_t n, int loc) { return elementwise(c, bb::EW_SIGMOID, x, x, nullptr, 0.f, n, loc); }
int bb_add_scaled(bb_ctx* c, float* out, const float* b, float s, size_t n, int loc) {
  return elementwise(c, bb::EW_ADD_SCALED, out, b, nullptr, s, n, loc);
}
int bb_add_assign(bb_ctx* c, float* a, const float* b, size_t n, int loc) {
  return elementwise(c, bb::EW_ADD_ASSIGN, a, b, nullptr, 0.f, n, loc);
}

int bb_rmsnorm(bb_ctx* c, const float* x, const float* gain, float eps, size_t n, size_t n_vec, float* out, int loc) {
  return guard([&] {
    need_ctx(c);
    need_loc(loc);
    set_device(c);
    with_io(c, loc, {{x, n * n_vec * 4, true, false}, {gain, n * 4, true, false}, {out, n * n_vec * 4, false, true}},
            [&](std::vector<void*>& d) {
              launch(c, bb::K_RMSNORM, [&] {
                return bb::launch_rmsnorm(c->stream, static_cast<const float*>(d[0]), static_cast<const float*>(d[1]), eps,
                                          n, n_vec, static_cast<float*>(d[2]));
              });
            });
  });
}

int bb_logits_from_hidden(bb_ctx* c, const bb_tensor* tok_embd, const float* gain, float eps, const float* h,
                          float* logits, int loc) {
  return guard([&] {
    need_ctx(c);
    need_loc(loc);
    need(tok_embd && gain && h && logits, BB_ERR_ARG, "null argument");
    need(tok_embd->ndims == 2, BB_ERR_SHAPE, "token_embd must be [hidden, vocab]");
    const size_t H = tok_embd->dims[0], V = tok_embd->dims[1];
    set_device(c);
    with_io(c, loc, {{h, H * 4, true, false}, {gain, H * 4, true, false}, {logits, V * 4, false, true}},
            [&](std::vector<void*>& d) {
              logits_dev(c, tok_embd, static_cast<const float*>(d[1]), eps, static_cast<const float*>(d[0]),
                         static_cast<float*>(d[2]));
            });
  });
}

int bb_moe_create(bb_ctx* c, const bb_tensor* router, const float* bias, const bb_tensor* gate, const bb_tensor* up,
                  const bb_tensor* down, int n_used, bb_moe** out) {
  return guard([&] {
    need_ctx(c);
    need(router && bias && gate && up && down && out, BB_ERR_ARG, "null argument");
    need(router->dtype == BB_F32, BB_ERR_DTYPE, "router (ffn_gate_inp) must be F32");
    need(router->ndims == 2, BB_ERR_SHAPE, "router must be [hidden, E]");
    const uint64_t H = router->dims[0], E = router->dims[1];
    need(gate->ndims == 3 && up->ndims == 3 && down->ndims == 3, BB_ERR_SHAPE, "expert tensors must be 3-D");
    const uint64_t F = gate->dims[1];
    need(gate->dims[0] == H && gate->dims[2] == E, BB_ERR_SHAPE, "gate_exps must be [hidden, ff, E]");
    need(up->dims[0] == H && up->dims[1] == F && up->dims[2] == E, BB_ERR_SHAPE, "up_exps must be [hidden, ff, E]");
    need(down->dims[0] == F && down->dims[1] == H && down->dims[2] == E, BB_ERR_SHAPE, "down_exps must be [ff, hidden, E]");
    for (const bb_tensor* t : {gate, up, down})
      need(t->dtype == BB_Q4_K || t->dtype == BB_Q6_K, BB_ERR_DTYPE, "expert tensors must be Q4_K or Q6_K");
    need(gate->dtype == up->dtype, BB_ERR_DTYPE, "gate_exps and up_exps must share a dtype");
    need(E >= 1 && E <= 32, BB_ERR_RANGE, "this build supports up to 32 experts");
    need(n_used >= 1 && n_used <= 8 && (uint64_t)n_used <= E, BB_ERR_RANGE, "n_used must be 1..min(8, E)");
    need(H % 256 == 0 && F % 256 == 0 && H >= 256 && F >= 256, BB_ERR_SHAPE, "hidden and ff must be multiples of 256");
    need(H <= (uint64_t)bb::GU_H_MAX && F <= (uint64_t)bb::DN_F_MAX, BB_ERR_RANGE,
         "hidden and ff above 2048 are not supported by the LDS-staged GEMV kernels");
    set_device(c);
    auto* m = new bb_moe();
    m->ctx = c;
    m->H = (int)H;
    m->F = (int)F;
    m->E = (int)E;
    m->K = n_used;
    size_t be, bgate, bup, bdown;
    block_of(gate->dtype, be, bgate);
    block_of(up->dtype, be, bup);
    block_of(down->dtype, be, bdown);
    const size_t stride_g = F * (H / 256) * bgate;  // model.rs:612-615
    const size_t stride_u = F * (H / 256) * bup;
    const size_t stride_d = H * (F / 256) * bdown;
    m->gu_dtype = (int)gate->dtype;
    m->dn_dtype = (int)down->dtype;
    m->stride_gu = (F / 32) * (H / 256) * bb::pack_tile_block_bytes(m->gu_dtype);
    m->stride_dn = (H / 64) * (F / 256) * bb::pack_tile_block_bytes(m->dn_dtype);
    try {
      m->bias_dev = static_cast<float*>(dev_alloc(E * 4));
      copy_to_dev(c, m->bias_dev, bias, E * 4, "bias upload");
      m->router_cm = static_cast<float*>(dev_alloc(E * H * 4));
      m->gu_packed = static_cast<uint8_t*>(dev_alloc(E * m->stride_gu));
      m->dn_packed = static_cast<uint8_t*>(dev_alloc(E * m->stride_dn));
      check_hip(bb::launch_router_chain_major(c->stream, reinterpret_cast<const float*>(router->dev), (int)H, (int)E,
                                              m->router_cm),
                "router layout");
      check_hip(bb::launch_pack_rows(c->stream, m->gu_dtype, gate->dev, up->dev, stride_g, stride_u, (int)F,
                                     (int)(H / 256), (int)E, m->gu_packed),
                "gate/up packing");
      check_hip(bb::launch_pack_rows(c->stream, m->dn_dtype, down->dev, nullptr, stride_d, 0, (int)H, (int)(F / 256),
                                     (int)E, m->dn_packed),
                "down packing");
      check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    } catch (...) {
      for (void* p : {(void*)m->bias_dev, (void*)m->router_cm, (void*)m->gu_packed, (void*)m->dn_packed})
        if (p) (void)hipFree(p);
      delete m;
      throw;
    }
    *out = m;
  });
}

int bb_moe_destroy(bb_moe* m) {
  return guard([&] {
    if (!m) return;
    set_device(m->ctx);
    (void)hipStreamSynchronize(m->ctx->stream);
    for (void* p : {(void*)m->bias_dev, (void*)m->router_cm, (void*)m->gu_packed, (void*)m->dn_packed})
      (void)hipFree(p);
    delete m;
  });
}

int bb_moe_forward(bb_ctx* c, bb_moe* m, const float* x, size_t T, float* out, int loc, bb_route_trace* tr) {
  return guard([&] {
    need_ctx(c);
    need(m != nullptr, BB_ERR_ARG, "null layer");
    need(m->ctx == c, BB_ERR_ARG, "layer belongs to another context");
    need_loc(loc);
    need(T >= 1, BB_ERR_ARG, "T must be >= 1");
    set_device(c);
    with_io(c, loc, {{x, T * m->H * 4, true, false}, {out, T * m->H * 4, false, true}}, [&](std::vector<void*>& d) {
      moe_forward_dev(c, m, static_cast<const float*>(d[0]), T, static_cast<float*>(d[1]), tr);
    });
  });
}

int bb_moe_forward_noalloc(bb_ctx* c, bb_moe* m, const float* x, size_t T, float* out) {
  return guard([&] {
    need_ctx(c);
    need(m != nullptr, BB_ERR_ARG, "null layer");
    need(m->ctx == c, BB_ERR_ARG, "layer belongs to another context");
    need(T >= 1, BB_ERR_ARG, "T must be >= 1");
    need_aligned(x, "x");
    need_aligned(out, "out");
    uint8_t* base = scratch_of(c->device);
    need(base != nullptr, BB_ERR_ARG, "no allocation-free scratch area on this device");
    set_device(c);
    // no events: profiling would take them from the context's pool, which may grow
    const bool prof = c->profile;
    c->profile = false;
    const WsRegion fixed{base, BB_NOALLOC_SCRATCH_BYTES};
    try {
      moe_forward_dev(c, m, x, T, out, nullptr, true, nullptr, &fixed);
    } catch (...) {
      c->profile = prof;
      throw;
    }
    c->profile = prof;
  });
}

int bb_dense_create(bb_ctx* c, const bb_tensor* gate, const bb_tensor* up, const bb_tensor* down, bb_dense** out) {
  return guard([&] {
    need_ctx(c);
    need(gate && up && down && out, BB_ERR_ARG, "null argument");
    need(gate->ndims == 2 && up->ndims == 2 && down->ndims == 2, BB_ERR_SHAPE, "dense weights must be 2-D");
    const uint64_t H = gate->dims[0], F = gate->dims[1];
    need(up->dims[0] == H && up->dims[1] == F, BB_ERR_SHAPE, "ffn_up must be [hidden, ff]");
    need(down->dims[0] == F && down->dims[1] == H, BB_ERR_SHAPE, "ffn_down must be [ff, hidden]");
    for (const bb_tensor* t : {gate, up, down})
      need(t->dtype == BB_Q4_K || t->dtype == BB_Q6_K, BB_ERR_DTYPE, "dense weights must be Q4_K or Q6_K");
    need(H % 256 == 0 && F % 256 == 0, BB_ERR_SHAPE, "hidden and ff must be multiples of 256");
    set_device(c);
    auto* d = new bb_dense();
    d->ctx = c;
    d->gate = gate;
    d->up = up;
    d->down = down;
    d->H = (int)H;
    d->F = (int)F;
    try {
      d->gu = pack_weights(c, gate, up, H, F);
      d->dn = pack_weights(c, down, nullptr, F, H);
    } catch (...) {
      free_packed(d->gu);
      delete d;
      throw;
    }
    *out = d;
  });
}

int bb_dense_destroy(bb_dense* d) {
  return guard([&] {
    if (!d) return;
    set_device(d->ctx);
    (void)hipStreamSynchronize(d->ctx->stream);
    free_packed(d->gu);
    free_packed(d->dn);
    delete d;
  });
}

int bb_dense_forward(bb_ctx* c, bb_dense* d, const float* x, size_t T, float* out, int loc) {
  return guard([&] {
    need_ctx(c);
    need(d != nullptr && d->ctx == c, BB_ERR_ARG, "bad dense layer");
    need_loc(loc);
    need(T >= 1, BB_ERR_ARG, "T must be >= 1");
    set_device(c);
    with_io(c, loc, {{x, T * d->H * 4, true, false}, {out, T * d->H * 4, false, true}}, [&](std::vector<void*>& dv) {
      dense_forward_dev(c, d, static_cast<const float*>(dv[0]), T, static_cast<float*>(dv[1]));
    });
  });
}

int bb_stack_create(bb_ctx* c, const bb_layer_desc* layers, size_t n_layers, float eps, bb_stack** out) {
  return guard([&] {
    need_ctx(c);
    need(layers && out && n_layers > 0, BB_ERR_ARG, "null argument");
    int H = -1;
    for (size_t i = 0; i < n_layers; ++i) {
      need((layers[i].moe != nullptr) != (layers[i].dense != nullptr), BB_ERR_ARG, "exactly one of moe/dense per layer");
      need(layers[i].ffn_norm != nullptr, BB_ERR_ARG, "ffn_norm is null");
      need(layers[i].moe ? layers[i].moe->ctx == c : layers[i].dense->ctx == c, BB_ERR_ARG,
           "a layer belongs to another context");
      const int h = layers[i].moe ? layers[i].moe->H : layers[i].dense->H;
      need(H < 0 || h == H, BB_ERR_SHAPE, "layers disagree on hidden size");
      H = h;
    }
    // the layer-boundary kernels hold a row of h per block in LDS
    need(H <= bb::GU_H_MAX, BB_ERR_RANGE, "the layer stack supports hidden sizes up to 2048");
    set_device(c);
    auto* s = new bb_stack();
    s->ctx = c;
    s->eps = eps;
    s->H = H;
    try {
      for (size_t i = 0; i < n_layers; ++i) {
        bb_layer_desc L = layers[i];
        float* g = static_cast<float*>(dev_alloc((size_t)H * 4));
        s->gains.push_back(g);
        copy_to_dev(c, g, layers[i].ffn_norm, (size_t)H * 4, "gain upload");
        L.ffn_norm = g;
        s->layers.push_back(L);
      }
    } catch (...) {
      for (float* g : s->gains) (void)hipFree(g);
      delete s;
      throw;
    }
    *out = s;
  });
}

int bb_stack_destroy(bb_stack* s) {
  return guard([&] {
    if (!s) return;
    set_device(s->ctx);
    (void)hipStreamSynchronize(s->ctx->stream);
    for (float* g : s->gains) (void)hipFree(g);
    for (void* p : {(void*)s->h, (void*)s->h2, (void*)s->normed, (void*)s->ffn, (void*)s->logits, (void*)s->xq_q,
                    (void*)s->xq_sx, (void*)s->xq_pairs})
      if (p) (void)hipFree(p);
    delete s;
  });
}

int bb_stack_forward(bb_ctx* c, bb_stack* s, const float* x, size_t T, float* h_out, int loc) {
  return guard([&] {
    need_ctx(c);
    need(s != nullptr && s->ctx == c, BB_ERR_ARG, "bad stack");
    need_loc(loc);
    need(T >= 1, BB_ERR_ARG, "T must be >= 1");
    set_device(c);
    const size_t H = s->H;
    if (T > s->cap_T) {
      check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
      for (void** p : {(void**)&s->h, (void**)&s->h2, (void**)&s->normed, (void**)&s->ffn, (void**)&s->logits,
                       (void**)&s->xq_q, (void**)&s->xq_sx, (void**)&s->xq_pairs}) {
        if (*p) (void)hipFree(*p);
        *p = nullptr;
      }
      s->cap_T = 0;
      s->h = static_cast<float*>(dev_alloc(T * H * 4));
      s->h2 = static_cast<float*>(dev_alloc(T * H * 4));
      s->normed = static_cast<float*>(dev_alloc(T * H * 4));
      s->ffn = static_cast<float*>(dev_alloc(T * H * 4));
      s->logits = static_cast<float*>(dev_alloc(T * 32 * 4));
      s->xq_q = static_cast<int8_t*>(dev_alloc(T * H));
      s->xq_sx = static_cast<float*>(dev_alloc(T * (H / 256) * 4));
      s->xq_pairs = static_cast<uint32_t*>(dev_alloc(T * (H / 256) * 12 * 4));
      s->cap_T = T;
    }
    with_io(c, loc, {{x, T * H * 4, true, false}, {h_out, T * H * 4, false, true}}, [&](std::vector<void*>& d) {
      float* h = s->h;       // the residual stream; at a boundary that routes, h_out is the other buffer
      float* h_alt = s->h2;
      check_hip(hipMemcpyAsync(h, d[0], T * H * 4, hipMemcpyDeviceToDevice, c->stream), "h copy");
      const size_t nl = s->layers.size();
      if (nl)
        launch(c, bb::K_RMSNORM,
               [&] { return bb::launch_rmsnorm(c->stream, h, s->layers[0].ffn_norm, s->eps, H, T, s->normed); });
      const PreRoute pre{s->logits, bb::XQBufs{s->xq_q, s->xq_sx, s->xq_pairs}};
      bool routed = false;  // the current layer's logits and XQ records are in pre
      for (size_t l = 0; l < nl; ++l) {
        const bb_layer_desc& L = s->layers[l];
        // the layer's FFN on normed, then h += its output and the next layer's rmsnorm, fused;
        // before an MoE layer of a few tokens on the GEMV path the same kernel also takes its
        // router logits
        const float* next_gain = l + 1 < nl ? s->layers[l + 1].ffn_norm : nullptr;
        const bb_moe* nm = l + 1 < nl ? s->layers[l + 1].moe : nullptr;
        const bool route_next = nm && T <= (size_t)bb::ROUTE_IN_GATEUP_MAX_T &&
                                T * (size_t)nm->K < c->batched_min_entries && H % 128 == 0 && nm->E <= 32 &&
                                nm->K <= 8;
        const float* slots = nullptr;
        const float* wts = nullptr;
        int K = 0;
        if (L.moe) {
          MoeWs w = moe_forward_dev(c, L.moe, s->normed, T, nullptr, nullptr, false, routed ? &pre : nullptr);
          slots = w.slots;
          wts = w.rb.wts;
          K = L.moe->K;
        } else {
          dense_forward_dev(c, L.dense, s->normed, T, s->ffn);
        }
        const float* ffn = L.moe ? nullptr : s->ffn;
        if (route_next) {
          launch(c, bb::K_RESIDUAL_ROUTE, [&] {
            return bb::launch_residual_norm_route(c->stream, h, h_alt, slots, wts, K, ffn, next_gain, s->eps, (int)H,
                                                  (int)T, s->normed, nm->router_cm, nm->E, s->logits, pre.xq);
          });
          std::swap(h, h_alt);
        } else {
          launch(c, bb::K_RESIDUAL_NORM, [&] {
            return bb::launch_residual_norm(c->stream, h, slots, wts, K, ffn, next_gain, s->eps, H, T, s->normed);
          });
        }
        routed = route_next;
      }
      check_hip(hipMemcpyAsync(d[1], h, T * H * 4, hipMemcpyDeviceToDevice, c->stream), "h copy");
    });
  });
}

// ---- decoder-layer operators -------------------------------------------------------------------

int bb_conv_step(bb_ctx* c, const float* state, const float* bx, const float* weight, size_t channels, size_t l_cache,
                 float* out, int loc) {
  return guard([&] {
    need_ctx(c);
    need_loc(loc);
    need(channels >= 1 && l_cache >= 1, BB_ERR_ARG, "channels and l_cache must be >= 1");
    need(channels * l_cache < (1u << 31), BB_ERR_RANGE, "conv too large");
    set_device(c);
    const size_t C = channels, L = l_cache;
    with_io(c, loc,
            {{state, (L - 1) * C * 4, true, false}, {bx, C * 4, true, false}, {weight, C * L * 4, true, false},
             {out, C * 4, false, true}},
            [&](std::vector<void*>& d) {
              launch(c, bb::K_CONV, [&] {
                return bb::launch_conv(c->stream, false, static_cast<const float*>(d[1]),
                                       static_cast<const float*>(d[0]), static_cast<const float*>(d[2]), (int)C, (int)L,
                                       1, static_cast<float*>(d[3]));
              });
            });
  });
}

int bb_conv_prefill(bb_ctx* c, float* state, const float* bx, const float* weight, size_t channels, size_t l_cache,
                    size_t n_tokens, float* out, int loc) {
  return guard([&] {
    need_ctx(c);
    need_loc(loc);
    need(channels >= 1 && l_cache >= 2, BB_ERR_ARG, "channels >= 1 and l_cache >= 2 required (conv.rs:58-66)");
    need(n_tokens >= 1, BB_ERR_ARG, "n_tokens must be >= 1");
    need(channels * (l_cache + n_tokens) < (1u << 31), BB_ERR_RANGE, "conv too large");
    set_device(c);
    const size_t C = channels, L = l_cache, T = n_tokens;
    with_io(c, loc,
            {{state, (L - 1) * C * 4, true, true}, {bx, T * C * 4, true, false}, {weight, C * L * 4, true, false},
             {out, T * C * 4, false, true}},
            [&](std::vector<void*>& d) {
              float* st = static_cast<float*>(d[0]);
              const float* b = static_cast<const float*>(d[1]);
              launch(c, bb::K_CONV, [&] {
                return bb::launch_conv(c->stream, false, b, st, static_cast<const float*>(d[2]), (int)C, (int)L, (int)T,
                                       static_cast<float*>(d[3]));
              });
              launch(c, bb::K_CONV_STATE,
                     [&] { return bb::launch_conv_state(c->stream, false, b, st, (int)C, (int)L, (int)T); });
            });
  });
}

int bb_softmax(bb_ctx* c, float* x, size_t n, size_t n_vec, int loc) {
  return guard([&] {
    need_ctx(c);
    need_loc(loc);
    need(n < (1u << 30) && n_vec < (1u << 30), BB_ERR_RANGE, "softmax too large");
    if (n == 0 || n_vec == 0) return;
    set_device(c);
    with_io(c, loc, {{x, n * n_vec * 4, true, true}}, [&](std::vector<void*>& d) {
      launch(c, bb::K_SOFTMAX, [&] { return bb::launch_softmax(c->stream, static_cast<float*>(d[0]), n, n_vec); });
    });
  });
}

int bb_attention_decode(bb_ctx* c, const float* q, const float* k, const float* v, size_t n_ctx, size_t n_heads,
                        size_t n_kv_heads, size_t head_dim, float* out, int loc) {
  return guard([&] {
    need_ctx(c);
    need_loc(loc);
    need(n_ctx >= 1 && n_heads >= 1 && n_kv_heads >= 1 && head_dim >= 1, BB_ERR_ARG, "sizes must be >= 1");
    need(n_heads % n_kv_heads == 0, BB_ERR_ARG, "n_heads must be a multiple of n_kv_heads");
    need(head_dim <= (size_t)bb::OPS_HD_MAX, BB_ERR_RANGE, "head_dim above 256");
    need(n_ctx * n_kv_heads * head_dim < (1u << 31) && n_ctx < (1u << 24), BB_ERR_RANGE, "context too large");
    set_device(c);
    const size_t QD = n_heads * head_dim, KVB = n_ctx * n_kv_heads * head_dim * 4;
    const float scale = 1.0f / std::sqrt(float(head_dim));
    with_io(c, loc, {{q, QD * 4, true, false}, {k, KVB, true, false}, {v, KVB, true, false}, {out, QD * 4, false, true}},
            [&](std::vector<void*>& d) {
              // (a float of slack after the rows: launch_attn_pv reads up to one past a row's end)
              float* scores = reinterpret_cast<float*>(ensure_ws(c, n_heads * n_ctx * 4 + 16));
              const int n0 = (int)n_ctx - 1;
              launch(c, bb::K_ATTN_SCORES, [&] {
                return bb::launch_attn_scores(c->stream, static_cast<const float*>(d[0]),
                                              static_cast<const float*>(d[1]), n0, 1, (int)n_heads, (int)n_kv_heads,
                                              (int)head_dim, scale, scores);
              });
              launch(c, bb::K_ATTN_PV, [&] {
                return bb::launch_attn_pv(c->stream, scores, static_cast<const float*>(d[2]), n0, 1, (int)n_heads,
                                          (int)n_kv_heads, (int)head_dim, static_cast<float*>(d[3]));
              });
            });
  });
}

int bb_rope_neox(bb_ctx* c, float* x, size_t head_dim, size_t n_vec, size_t pos, float freq_base, int loc) {
  return guard([&] {
    need_ctx(c);
    need_loc(loc);
    need(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= (size_t)bb::OPS_HD_MAX, BB_ERR_ARG,
         "head_dim must be even and at most 256");
    need(n_vec >= 1 && n_vec < (1u << 16), BB_ERR_RANGE, "n_vec must be in 1..65535");
    set_device(c);
    std::vector<float2> tab;
    rope_rows(tab, pos, 1, head_dim, freq_base);
    with_io(c, loc, {{x, n_vec * head_dim * 4, true, true}}, [&](std::vector<void*>& d) {
      auto* t = reinterpret_cast<float2*>(ensure_ws(c, tab.size() * sizeof(float2)));
      check_hip(hipMemcpyAsync(t, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice, c->stream),
                "RoPE row upload");
      // n_vec heads of one position: the heads are the kernel's head axis of one token
      launch(c, bb::K_NORM_ROPE, [&] {
        return bb::launch_norm_rope(c->stream, static_cast<float*>(d[0]), 1, (int)n_vec, (int)head_dim, nullptr, 0.0f,
                                    t);
      });
      check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");  // tab is a host temporary
    });
  });
}

int bb_conv_op_create(bb_ctx* c, const bb_tensor* in_proj, const float* conv_w, size_t l_cache,
                      const bb_tensor* out_proj, bb_conv_op** out) {
  return guard([&] {
    need_ctx(c);
    need(in_proj && out_proj && conv_w && out, BB_ERR_ARG, "null argument");
    need(l_cache >= 2 && l_cache <= 64, BB_ERR_ARG, "l_cache must be in 2..64");
    need(in_proj->ndims == 2, BB_ERR_SHAPE, "in_proj must be 2-D");
    const uint64_t H = in_proj->dims[0];
    need_proj(in_proj, H, 3 * H, "shortconv.in_proj");
    need_proj(out_proj, H, H, "shortconv.out_proj");
    need(H % 256 == 0 && H * 3 * 64 < (1u << 31), BB_ERR_SHAPE, "hidden must be a multiple of 256");
    set_device(c);
    auto* op = new bb_conv_op();
    op->ctx = c;
    op->in_proj = in_proj;
    op->out_proj = out_proj;
    op->H = (int)H;
    op->L = (int)l_cache;
    try {
      op->conv_w = upload_f32(c, conv_w, H * l_cache);
      op->in_p = pack_weights(c, in_proj, nullptr, H, 3 * H);
      op->out_p = pack_weights(c, out_proj, nullptr, H, H);
    } catch (...) {
      if (op->conv_w) (void)hipFree(op->conv_w);
      free_packed(op->in_p);
      delete op;
      throw;
    }
    *out = op;
  });
}

int bb_conv_op_destroy(bb_conv_op* op) {
  return guard([&] {
    if (!op) return;
    set_device(op->ctx);
    (void)hipStreamSynchronize(op->ctx->stream);
    (void)hipFree(op->conv_w);
    free_packed(op->in_p);
    free_packed(op->out_p);
    delete op;
  });
}

int bb_conv_op_forward(bb_ctx* c, bb_conv_op* op, float* state, const float* x, size_t T, float* out, int loc) {
  return guard([&] {
    need_ctx(c);
    need(op != nullptr && op->ctx == c, BB_ERR_ARG, "bad conv operator");
    need_loc(loc);
    need(T >= 1 && T <= (size_t)bb::PF_MAX_ENTRIES, BB_ERR_RANGE, "T must be in 1..32768");
    set_device(c);
    const size_t H = op->H;
    with_io(c, loc,
            {{state, (op->L - 1) * H * 4, true, true}, {x, T * H * 4, true, false}, {out, T * H * 4, false, true}},
            [&](std::vector<void*>& d) {
              conv_forward_dev(c, op, static_cast<float*>(d[0]), static_cast<const float*>(d[1]), T,
                               static_cast<float*>(d[2]));
            });
  });
}

int bb_kv_cache_create(bb_ctx* c, size_t kv_dim, size_t capacity, bb_kv_cache** out) {
  return guard([&] {
    need_ctx(c);
    need(out != nullptr && kv_dim >= 1 && capacity >= 1, BB_ERR_ARG, "bad argument");
    need(kv_dim * capacity < (1u << 29), BB_ERR_RANGE, "cache above 2 GB per array");
    set_device(c);
    auto* kv = new bb_kv_cache();
    kv->ctx = c;
    kv->kv_dim = kv_dim;
    kv->cap = capacity;
    kv->n = 0;
    try {
      kv->k = static_cast<float*>(dev_alloc(kv_dim * capacity * 4));
      kv->v = static_cast<float*>(dev_alloc(kv_dim * capacity * 4));
    } catch (...) {
      if (kv->k) (void)hipFree(kv->k);
      delete kv;
      throw;
    }
    *out = kv;
  });
}

int bb_kv_cache_destroy(bb_kv_cache* kv) {
  return guard([&] {
    if (!kv) return;
    set_device(kv->ctx);
    (void)hipFree(kv->k);
    (void)hipFree(kv->v);
    delete kv;
  });
}

int bb_kv_cache_length(const bb_kv_cache* kv, size_t* n) {
  return guard([&] {
    need(kv != nullptr && n != nullptr, BB_ERR_ARG, "null argument");
    *n = kv->n;
  });
}

int bb_kv_cache_read(bb_ctx* c, const bb_kv_cache* kv, float* k, float* v, int loc) {
  return guard([&] {
    need_ctx(c);
    need(kv != nullptr && kv->ctx == c, BB_ERR_ARG, "bad cache");
    need_loc(loc);
    set_device(c);
    const size_t bytes = kv->n * kv->kv_dim * 4;
    if (bytes == 0) return;
    need(k != nullptr && v != nullptr, BB_ERR_ARG, "null output");
    const hipMemcpyKind kind = loc == BB_LOC_HOST ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
    check_hip(hipMemcpyAsync(k, kv->k, bytes, kind, c->stream), "cache copy");
    check_hip(hipMemcpyAsync(v, kv->v, bytes, kind, c->stream), "cache copy");
    if (loc == BB_LOC_HOST) check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  });
}

int bb_kv_cache_evict_front(bb_ctx* c, bb_kv_cache* kv, size_t n) {
  return guard([&] {
    need_ctx(c);
    need(kv != nullptr && kv->ctx == c, BB_ERR_ARG, "bad cache");
    set_device(c);
    // a history shorter than n positions is left as it is (cache.rs:44: `if k.len() >= drop`)
    if (n == 0 || n > kv->n) return;
    if (n == kv->n) {
      kv->n = 0;
      return;
    }
    // positions n.. move to the front (device copies through a staging area: the ranges overlap)
    const size_t keep = (kv->n - n) * kv->kv_dim * 4;
    auto* tmp = ensure_ws(c, keep);
    for (float* a : {kv->k, kv->v}) {
      check_hip(hipMemcpyAsync(tmp, a + n * kv->kv_dim, keep, hipMemcpyDeviceToDevice, c->stream), "cache copy");
      check_hip(hipMemcpyAsync(a, tmp, keep, hipMemcpyDeviceToDevice, c->stream), "cache copy");
    }
    kv->n -= n;
  });
}

int bb_attn_op_create(bb_ctx* c, const bb_tensor* q, const bb_tensor* k, const bb_tensor* v, const bb_tensor* o,
                      const float* q_norm, const float* k_norm, size_t n_heads, size_t n_kv_heads, float eps,
                      float freq_base, bb_attn_op** out) {
  return guard([&] {
    need_ctx(c);
    need(q && k && v && o && q_norm && k_norm && out, BB_ERR_ARG, "null argument");
    need(n_heads >= 1 && n_kv_heads >= 1 && n_heads % n_kv_heads == 0, BB_ERR_ARG,
         "n_heads must be a positive multiple of n_kv_heads");
    need(q->ndims == 2, BB_ERR_SHAPE, "attn_q must be 2-D");
    const uint64_t H = q->dims[0], QD = q->dims[1];
    need(QD % n_heads == 0, BB_ERR_SHAPE, "attn_q's output size must be n_heads * head_dim");
    const uint64_t HD = QD / n_heads, KV = n_kv_heads * HD;
    need(HD >= 2 && HD % 2 == 0 && HD <= (uint64_t)bb::OPS_HD_MAX, BB_ERR_RANGE, "head_dim must be even and <= 256");
    need_proj(q, H, QD, "attn_q");
    need_proj(k, H, KV, "attn_k");
    need_proj(v, H, KV, "attn_v");
    need_proj(o, QD, H, "attn_output");
    set_device(c);
    auto* op = new bb_attn_op();
    op->ctx = c;
    op->q = q;
    op->k = k;
    op->v = v;
    op->o = o;
    op->H = (int)H;
    op->NH = (int)n_heads;
    op->NKV = (int)n_kv_heads;
    op->HD = (int)HD;
    op->eps = eps;
    op->freq_base = freq_base;
    op->scale = 1.0f / std::sqrt(float(HD));  // attention.rs:35
    try {
      op->q_norm = upload_f32(c, q_norm, HD);
      op->k_norm = upload_f32(c, k_norm, HD);
      ensure_rope(c, op, 4096);
      op->q_p = pack_weights(c, q, nullptr, H, QD);
      op->k_p = pack_weights(c, k, nullptr, H, KV);
      op->v_p = pack_weights(c, v, nullptr, H, KV);
      op->o_p = pack_weights(c, o, nullptr, QD, H);
    } catch (...) {
      if (op->q_norm) (void)hipFree(op->q_norm);
      if (op->k_norm) (void)hipFree(op->k_norm);
      if (op->rope) (void)hipFree(op->rope);
      for (bb::PackedW* p : {&op->q_p, &op->k_p, &op->v_p, &op->o_p}) free_packed(*p);
      delete op;
      throw;
    }
    *out = op;
  });
}

int bb_attn_op_destroy(bb_attn_op* op) {
  return guard([&] {
    if (!op) return;
    set_device(op->ctx);
    (void)hipStreamSynchronize(op->ctx->stream);
    (void)hipFree(op->q_norm);
    (void)hipFree(op->k_norm);
    if (op->rope) (void)hipFree(op->rope);
    for (bb::PackedW* p : {&op->q_p, &op->k_p, &op->v_p, &op->o_p}) free_packed(*p);
    delete op;
  });
}

int bb_attn_op_forward(bb_ctx* c, bb_attn_op* op, bb_kv_cache* kv, size_t pos0, const float* x, size_t T, float* out,
                       int loc) {
  return guard([&] {
    need_ctx(c);
    need(op != nullptr && op->ctx == c, BB_ERR_ARG, "bad attention operator");
    need(kv != nullptr && kv->ctx == c, BB_ERR_ARG, "bad cache");
    need_loc(loc);
    need(kv->kv_dim == (size_t)op->NKV * op->HD, BB_ERR_SHAPE, "cache kv_dim must be n_kv_heads * head_dim");
    need(T >= 1 && T <= (size_t)bb::PF_MAX_ENTRIES, BB_ERR_RANGE, "T must be in 1..32768");
    need(kv->n + T <= kv->cap, BB_ERR_RANGE, "the cache is full (evict positions first, cache.rs:40-50)");
    need(pos0 + T < (1u << 24), BB_ERR_RANGE, "position beyond 2^24");
    set_device(c);
    const size_t H = op->H;
    with_io(c, loc, {{x, T * H * 4, true, false}, {out, T * H * 4, false, true}}, [&](std::vector<void*>& d) {
      attn_forward_dev(c, op, kv, pos0, static_cast<const float*>(d[0]), T, static_cast<float*>(d[1]));
    });
  });
}

// ---- the decoder ---------------------------------------------------------------------------------
namespace {

// Cache::kv_len (cache.rs:32-35): the longest attention layer's history.
size_t cache_kv_len(const bb_cache* k) {
  size_t n = 0;
  for (const bb_kv_cache* kv : k->kv)
    if (kv) n = std::max(n, kv->n);
  return n;
}

// Room for `want` positions in one layer's KV history: the reference appends to growing Vecs,
// so a full cache grows (to at least twice its capacity) instead of failing. The n cached
// positions are copied into the new arrays on the context's stream, which is drained before
// the old arrays are freed.
void kv_reserve(bb_ctx* c, bb_kv_cache* kv, size_t want) {
  if (want <= kv->cap) return;
  const size_t cap = std::max(want, 2 * kv->cap);
  need(kv->kv_dim * cap < (1u << 29), BB_ERR_RANGE, "KV cache above 2 GB per array");
  float* nk = static_cast<float*>(dev_alloc(kv->kv_dim * cap * 4));
  float* nv = nullptr;
  try {
    nv = static_cast<float*>(dev_alloc(kv->kv_dim * cap * 4));
  } catch (...) {
    (void)hipFree(nk);
    throw;
  }
  const size_t bytes = kv->n * kv->kv_dim * 4;
  if (bytes) {
    check_hip(hipMemcpyAsync(nk, kv->k, bytes, hipMemcpyDeviceToDevice, c->stream), "cache copy");
    check_hip(hipMemcpyAsync(nv, kv->v, bytes, hipMemcpyDeviceToDevice, c->stream), "cache copy");
  }
  check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  (void)hipFree(kv->k);
  (void)hipFree(kv->v);
  kv->k = nk;
  kv->v = nv;
  kv->cap = cap;
}

void model_buffers(bb_ctx* c, bb_model* m, size_t T) {
  if (T <= m->cap_T) return;
  check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  for (void** p : {(void**)&m->h, (void**)&m->normed, (void**)&m->tmp, (void**)&m->nq.q, (void**)&m->nq.scales,
                   (void**)&m->nq.sums, (void**)&m->h2, (void**)&m->logits, (void**)&m->xq.q, (void**)&m->xq.sx,
                   (void**)&m->xq.pairs}) {
    if (*p) (void)hipFree(*p);
    *p = nullptr;
  }
  m->cap_T = 0;
  const size_t H = m->H;
  m->h = static_cast<float*>(dev_alloc(T * H * 4));
  m->normed = static_cast<float*>(dev_alloc(T * H * 4));
  m->tmp = static_cast<float*>(dev_alloc(T * H * 4));
  if (H % 256 == 0) {
    m->nq.q = static_cast<int8_t*>(dev_alloc(T * H));
    m->nq.scales = static_cast<float*>(dev_alloc(T * H / 256 * 4));
    m->nq.sums = static_cast<int32_t*>(dev_alloc(T * H / 32 * 4));
  }
  if (H % 256 == 0) {
    // (h2 as large as h: the two trade places at a routing boundary; the logits and XQ records
    // serve calls of at most ROUTE_IN_GATEUP_MAX_T tokens)
    constexpr size_t TR = bb::ROUTE_IN_GATEUP_MAX_T;
    m->h2 = static_cast<float*>(dev_alloc(T * H * 4));
    m->logits = static_cast<float*>(dev_alloc(TR * 32 * 4));
    m->xq.q = static_cast<int8_t*>(dev_alloc(TR * H));
    m->xq.sx = static_cast<float*>(dev_alloc(TR * (H / 256) * 4));
    m->xq.pairs = static_cast<uint32_t*>(dev_alloc(TR * (H / 256) * 12 * 4));
  }
  m->cap_T = T;
}

// The token ids of one call, checked and copied to the device once. The stream is drained
// first: the buffer is reused by every call, and an earlier call's embedding may still read it
// (a copy from pageable host memory is not guaranteed to wait for the stream's earlier work).
const uint32_t* model_tokens(bb_ctx* c, bb_model* m, const uint32_t* host, size_t n) {
  for (size_t i = 0; i < n; ++i) need(host[i] < m->vocab, BB_ERR_ARG, "token id beyond the vocabulary");
  check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  if (n > m->tok_cap) {
    if (m->tok) (void)hipFree(m->tok);
    m->tok = nullptr;
    m->tok_cap = 0;
    m->tok = static_cast<uint32_t*>(dev_alloc(n * 4));
    m->tok_cap = n;
  }
  copy_to_dev(c, m->tok, host, n * 4, "token copy");
  return m->tok;
}

// Model::run_layers (T == 1, model.rs:105-130) / run_layers_batch (T > 1, :146-181): embeds
// the tokens (device ids) at positions k->pos.., runs every layer (updating the cache's conv
// states and KV histories) and leaves the final hidden states in m->h.
void model_run_dev(bb_ctx* c, bb_model* m, bb_cache* k, const uint32_t* tokens, size_t T) {
  for (bb_kv_cache* kv : k->kv)
    if (kv) kv_reserve(c, kv, kv->n + T);
  model_buffers(c, m, T);
  const size_t H = m->H;
  launch(c, bb::K_EMBED, [&] {
    return bb::launch_embed(c->stream, m->tok_embd->dev, (int)m->tok_embd->dtype, m->row_bytes, tokens, (int)T, (int)H,
                            m->h);
  });
  // Each layer boundary (h += sub-layer output, then the next rmsnorm) is one launch of
  // k_residual_norm, which also writes the normed rows' Q8 when the next sub-layer projects
  // them (conv, attention, dense FFN; the MoE route quantises its input itself), or, before an
  // MoE layer of a few tokens, of k_residual_norm_route, which also takes the layer's router
  // logits and XQ records.
  const bool fused = H <= (size_t)bb::GU_H_MAX && m->nq.q;
  auto boundary = [&](const float* gain, bool q8) {
    if (fused) {
      launch(c, bb::K_RESIDUAL_NORM, [&] {
        return bb::launch_residual_norm(c->stream, m->h, nullptr, nullptr, 0, m->tmp, gain, m->eps, H, T, m->normed,
                                        q8 && gain ? m->nq : bb::Q8Bufs{});
      });
      return;
    }
    launch(c, bb::K_ELEMWISE, [&] {
      return bb::launch_elementwise(c->stream, bb::EW_ADD_ASSIGN, m->h, m->tmp, nullptr, 0.0f, T * H);
    });
    if (gain) launch(c, bb::K_RMSNORM, [&] { return bb::launch_rmsnorm(c->stream, m->h, gain, m->eps, H, T, m->normed); });
  };
  const bb::Q8Bufs* nq = fused ? &m->nq : nullptr;
  const size_t n_layers = m->layers.size();
  if (fused)
    launch(c, bb::K_RMSNORM, [&] {
      return bb::launch_rmsnorm_q8(c->stream, m->h, m->layers[0].attn_norm, m->eps, H, T, m->normed, m->nq);
    });
  else
    launch(c, bb::K_RMSNORM, [&] {
      return bb::launch_rmsnorm(c->stream, m->h, m->layers[0].attn_norm, m->eps, H, T, m->normed);
    });
  for (size_t i = 0; i < n_layers; ++i) {
    auto& L = m->layers[i];
    if (L.conv) conv_forward_dev(c, L.conv, k->conv[i], m->normed, T, m->tmp, nq);
    else attn_forward_dev(c, L.attn, k->kv[i], k->pos, m->normed, T, m->tmp, nq);
    // before an MoE layer of a few tokens on the GEMV path the boundary also takes the layer's
    // router logits and its input's XQ records, and the gate/up GEMV only gates
    const bb_moe* mo = L.moe;
    const bool route_here = fused && mo && m->h2 && T <= (size_t)bb::ROUTE_IN_GATEUP_MAX_T &&
                            T * (size_t)mo->K < c->batched_min_entries && H % 128 == 0 && mo->E <= 32 &&
                            mo->K <= 8;
    if (route_here) {
      launch(c, bb::K_RESIDUAL_ROUTE, [&] {
        return bb::launch_residual_norm_route(c->stream, m->h, m->h2, nullptr, nullptr, 0, m->tmp, L.ffn_norm, m->eps,
                                              (int)H, (int)T, m->normed, mo->router_cm, mo->E, m->logits, m->xq);
      });
      std::swap(m->h, m->h2);
      const PreRoute pre{m->logits, m->xq};
      moe_forward_dev(c, L.moe, m->normed, T, m->tmp, nullptr, true, &pre);
    } else {
      boundary(L.ffn_norm, L.dense != nullptr);
      if (L.moe) moe_forward_dev(c, L.moe, m->normed, T, m->tmp, nullptr);
      else dense_forward_dev(c, L.dense, m->normed, T, m->tmp, nq);
    }
    boundary(i + 1 < n_layers ? m->layers[i + 1].attn_norm : nullptr, true);
  }
  k->pos += T;
}

// Cache::evict_front (cache.rs:40-50) on every attention layer.
void cache_evict(bb_ctx* c, bb_cache* k, size_t n) {
  if (n == 0) return;
  for (bb_kv_cache* kv : k->kv)
    if (kv) check_code(bb_kv_cache_evict_front(c, kv, n));
}

// Cache::new (cache.rs:21-28) for the layers of m: conv states zeroed, empty KV histories.
void cache_clear(bb_ctx* c, bb_cache* k) {
  const bb_model* m = k->model;
  for (size_t i = 0; i < m->layers.size(); ++i) {
    if (k->conv[i]) {
      float* st = k->conv[i];
      const size_t n = (size_t)(m->layers[i].conv->L - 1) * m->H;
      launch(c, bb::K_ELEMWISE, [&] { return bb::launch_zero(c->stream, st, n); });
    }
    if (k->kv[i]) k->kv[i]->n = 0;
  }
  k->pos = 0;
}

void cache_free(bb_cache* k) {
  for (float* p : k->conv)
    if (p) (void)hipFree(p);
  for (bb_kv_cache* kv : k->kv)
    if (kv) (void)bb_kv_cache_destroy(kv);
  delete k;
}

// A cache of m's layout: conv states and KV histories allocated, contents not yet set.
bb_cache* cache_alloc(bb_ctx* c, const bb_model* m, size_t kv_capacity) {
  auto* k = new bb_cache();
  k->ctx = c;
  k->model = m;
  k->conv.assign(m->layers.size(), nullptr);
  k->kv.assign(m->layers.size(), nullptr);
  try {
    for (size_t i = 0; i < m->layers.size(); ++i) {
      const auto& L = m->layers[i];
      if (L.conv) k->conv[i] = static_cast<float*>(dev_alloc((size_t)(L.conv->L - 1) * m->H * 4));
      else check_code(bb_kv_cache_create(c, (size_t)L.attn->NKV * L.attn->HD, kv_capacity, &k->kv[i]));
    }
  } catch (...) {
    cache_free(k);
    throw;
  }
  return k;
}

void need_model_cache(bb_ctx* c, const bb_model* m, const bb_cache* k) {
  need(m != nullptr && m->ctx == c, BB_ERR_ARG, "bad model");
  need(k != nullptr && k->model == m && k->ctx == c, BB_ERR_ARG, "the cache belongs to another model or context");
}

}  // namespace

int bb_model_create(bb_ctx* c, const bb_tensor* token_embd, const float* final_norm, const bb_decoder_layer* layers,
                    size_t n_layers, float eps, bb_model** out) {
  return guard([&] {
    need_ctx(c);
    need(token_embd && final_norm && layers && out && n_layers > 0, BB_ERR_ARG, "null argument");
    need(token_embd->ndims == 2, BB_ERR_SHAPE, "token_embd must be [hidden, vocab]");
    const size_t H = token_embd->dims[0], V = token_embd->dims[1];
    size_t be, bb_;
    need(block_of(token_embd->dtype, be, bb_) && H % be == 0, BB_ERR_DTYPE, "unsupported token_embd dtype or shape");
    for (size_t i = 0; i < n_layers; ++i) {
      const bb_decoder_layer& D = layers[i];
      need(D.attn_norm && D.ffn_norm, BB_ERR_ARG, "layer norms must be set");
      need((D.conv != nullptr) != (D.attn != nullptr), BB_ERR_ARG, "exactly one of conv/attn per layer");
      need((D.moe != nullptr) != (D.dense != nullptr), BB_ERR_ARG, "exactly one of moe/dense per layer");
      const int oh = D.conv ? D.conv->H : D.attn->H;
      const int fh = D.moe ? D.moe->H : D.dense->H;
      need(oh == (int)H && fh == (int)H, BB_ERR_SHAPE, "layers disagree with token_embd on the hidden size");
      need((D.conv ? D.conv->ctx : D.attn->ctx) == c && (D.moe ? D.moe->ctx : D.dense->ctx) == c, BB_ERR_ARG,
           "a layer belongs to another context");
    }
    set_device(c);
    auto* m = new bb_model();
    m->ctx = c;
    m->tok_embd = token_embd;
    m->eps = eps;
    m->H = (int)H;
    m->vocab = V;
    m->row_bytes = H / be * bb_;
    try {
      m->final_norm = upload_f32(c, final_norm, H);
      for (size_t i = 0; i < n_layers; ++i) {
        const bb_decoder_layer& D = layers[i];
        bb_model::Layer L{};
        L.conv = D.conv;
        L.attn = D.attn;
        L.moe = D.moe;
        L.dense = D.dense;
        m->layers.push_back(L);
        bb_model::Layer& B = m->layers.back();
        B.attn_norm = upload_f32(c, D.attn_norm, H);
        B.ffn_norm = upload_f32(c, D.ffn_norm, H);
      }
    } catch (...) {
      (void)bb_model_destroy(m);
      throw;
    }
    *out = m;
  });
}

int bb_model_destroy(bb_model* m) {
  return guard([&] {
    if (!m) return;
    set_device(m->ctx);
    (void)hipStreamSynchronize(m->ctx->stream);
    for (auto& L : m->layers) {
      if (L.attn_norm) (void)hipFree(L.attn_norm);
      if (L.ffn_norm) (void)hipFree(L.ffn_norm);
    }
    for (void* p : {(void*)m->final_norm, (void*)m->h, (void*)m->normed, (void*)m->tmp, (void*)m->tok,
                    (void*)m->nq.q, (void*)m->nq.scales, (void*)m->nq.sums, (void*)m->h2, (void*)m->logits,
                    (void*)m->xq.q, (void*)m->xq.sx, (void*)m->xq.pairs})
      if (p) (void)hipFree(p);
    bb::free_owned(m->owned);
    delete m;
  });
}

int bb_cache_create(bb_ctx* c, const bb_model* m, size_t kv_capacity, bb_cache** out) {
  return guard([&] {
    need_ctx(c);
    need(m != nullptr && m->ctx == c, BB_ERR_ARG, "bad model");
    need(out != nullptr, BB_ERR_ARG, "null argument");
    need(kv_capacity >= 1, BB_ERR_ARG, "kv_capacity must be >= 1");
    set_device(c);
    bb_cache* k = cache_alloc(c, m, kv_capacity);
    try {
      cache_clear(c, k);
      check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    } catch (...) {
      cache_free(k);
      throw;
    }
    *out = k;
  });
}

int bb_cache_clone(bb_ctx* c, const bb_cache* src, bb_cache** out) {
  return guard([&] {
    need_ctx(c);
    need(src != nullptr && src->ctx == c, BB_ERR_ARG, "bad cache");
    need(out != nullptr, BB_ERR_ARG, "null argument");
    set_device(c);
    const bb_model* m = src->model;
    size_t cap = 1;
    for (const bb_kv_cache* kv : src->kv)
      if (kv) cap = std::max(cap, kv->cap);
    bb_cache* k = cache_alloc(c, m, cap);
    try {
      for (size_t i = 0; i < m->layers.size(); ++i) {
        if (src->conv[i])
          check_hip(hipMemcpyAsync(k->conv[i], src->conv[i], (size_t)(m->layers[i].conv->L - 1) * m->H * 4,
                                   hipMemcpyDeviceToDevice, c->stream),
                    "cache copy");
        if (src->kv[i]) {
          const bb_kv_cache* a = src->kv[i];
          bb_kv_cache* b = k->kv[i];
          const size_t bytes = a->n * a->kv_dim * 4;
          if (bytes) {
            check_hip(hipMemcpyAsync(b->k, a->k, bytes, hipMemcpyDeviceToDevice, c->stream), "cache copy");
            check_hip(hipMemcpyAsync(b->v, a->v, bytes, hipMemcpyDeviceToDevice, c->stream), "cache copy");
          }
          b->n = a->n;
        }
      }
      k->pos = src->pos;
      check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    } catch (...) {
      cache_free(k);
      throw;
    }
    *out = k;
  });
}

int bb_cache_destroy(bb_cache* k) {
  return guard([&] {
    if (!k) return;
    set_device(k->ctx);
    (void)hipStreamSynchronize(k->ctx->stream);
    cache_free(k);
  });
}

int bb_cache_reset(bb_ctx* c, bb_cache* k) {
  return guard([&] {
    need_ctx(c);
    need(k != nullptr && k->ctx == c, BB_ERR_ARG, "bad cache");
    set_device(c);
    cache_clear(c, k);
  });
}

int bb_cache_position(const bb_cache* k, size_t* pos) {
  return guard([&] {
    need(k != nullptr && pos != nullptr, BB_ERR_ARG, "null argument");
    *pos = k->pos;
  });
}

int bb_cache_kv_length(const bb_cache* k, size_t* n) {
  return guard([&] {
    need(k != nullptr && n != nullptr, BB_ERR_ARG, "null argument");
    *n = cache_kv_len(k);
  });
}

int bb_cache_evict_front(bb_ctx* c, bb_cache* k, size_t n) {
  return guard([&] {
    need_ctx(c);
    need(k != nullptr && k->ctx == c, BB_ERR_ARG, "bad cache");
    set_device(c);
    cache_evict(c, k, n);
  });
}

int bb_cache_layer_state(bb_ctx* c, const bb_cache* k, size_t layer, float* conv_state, float* kk, float* v, int loc) {
  return guard([&] {
    need_ctx(c);
    need(k != nullptr && k->ctx == c && layer < k->conv.size(), BB_ERR_ARG, "bad cache or layer");
    need_loc(loc);
    set_device(c);
    const bb_model* m = k->model;
    const hipMemcpyKind kind = loc == BB_LOC_HOST ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
    if (k->conv[layer] && conv_state)
      check_hip(hipMemcpyAsync(conv_state, k->conv[layer], (size_t)(m->layers[layer].conv->L - 1) * m->H * 4, kind,
                               c->stream),
                "copy");
    const bb_kv_cache* kv = k->kv[layer];
    if (kv && kv->n) {
      const size_t bytes = kv->n * kv->kv_dim * 4;
      if (kk) check_hip(hipMemcpyAsync(kk, kv->k, bytes, kind, c->stream), "copy");
      if (v) check_hip(hipMemcpyAsync(v, kv->v, bytes, kind, c->stream), "copy");
    }
    check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  });
}

int bb_model_run_layers(bb_ctx* c, bb_model* m, const uint32_t* tokens, size_t T, bb_cache* k, float* h_out,
                        int loc) {
  return guard([&] {
    need_ctx(c);
    need_model_cache(c, m, k);
    need_loc(loc);
    need(tokens != nullptr && T >= 1 && T <= (size_t)bb::PF_MAX_ENTRIES / 8, BB_ERR_RANGE, "T must be in 1..4096");
    set_device(c);
    const size_t H = m->H;
    with_io(c, loc, {{h_out, T * H * 4, false, true}}, [&](std::vector<void*>& d) {
      model_run_dev(c, m, k, model_tokens(c, m, tokens, T), T);
      if (h_out) check_hip(hipMemcpyAsync(d[0], m->h, T * H * 4, hipMemcpyDeviceToDevice, c->stream), "h copy");
    });
  });
}

int bb_model_forward_step(bb_ctx* c, bb_model* m, uint32_t token, bb_cache* k, float* logits, int loc) {
  return guard([&] {
    need_ctx(c);
    need_model_cache(c, m, k);
    need_loc(loc);
    set_device(c);
    with_io(c, loc, {{logits, m->vocab * 4, false, true}}, [&](std::vector<void*>& d) {
      model_run_dev(c, m, k, model_tokens(c, m, &token, 1), 1);
      logits_dev(c, m->tok_embd, m->final_norm, m->eps, m->h, static_cast<float*>(d[0]));
    });
  });
}

// Every token id is checked before anything runs, and a KV history that would overflow grows
// (kv_reserve), so the call does not stop half-way with the cache partly advanced.
int bb_model_absorb(bb_ctx* c, bb_model* m, bb_cache* k, const uint32_t* tokens, size_t n, size_t max_context) {
  return guard([&] {
    need_ctx(c);
    need_model_cache(c, m, k);
    need(tokens != nullptr || n == 0, BB_ERR_ARG, "null tokens");
    set_device(c);
    const size_t chunk = 512;  // agent.rs:31 PREFILL_CHUNK
    if (n == 0) return;
    const uint32_t* dt = model_tokens(c, m, tokens, n);
    if (cache_kv_len(k) + n <= max_context) {
      for (bb_kv_cache* kv : k->kv)
        if (kv) kv_reserve(c, kv, kv->n + n);
      for (size_t i = 0; i < n; i += chunk) model_run_dev(c, m, k, dt + i, std::min(chunk, n - i));
    } else {
      for (bb_kv_cache* kv : k->kv)
        if (kv) kv_reserve(c, kv, std::max(kv->n, max_context) + 1);
      for (size_t i = 0; i < n; ++i) {
        model_run_dev(c, m, k, dt + i, 1);
        const size_t len = cache_kv_len(k);
        if (len > max_context) cache_evict(c, k, len - max_context);
      }
    }
    check_hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  });
}

}  // extern "C"
