// Host side of the multi-row forward (rows_kernel.h): plan (geometry checks,
// per-layer pointer table, kernel instance), state (flags, epoch, partial
// sums and activation rows) and the launch.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <vector>

#include "kernels.h"
#include "rows.h"
#include "rows_kernel.h"

namespace rtg {

namespace {
constexpr size_t kHead = rows_state_head_bytes();  // flags, epoch, counters, error word
constexpr size_t kAlign = 256;
size_t align_up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

}  // namespace

struct RowsPlan {
  int d = 0, H = 0, V = 0, L = 0, P = 0;
  const void* kernel[2] = {nullptr, nullptr};  // shared regions, layered (FRESH) regions
  rk::RLayer* layers_dev = nullptr;
  rk::RParams base{};
  size_t p0q = 0, p0f = 0, p1 = 0;  // floats of a layer's c_attn / c_fc partials, of P1
};

namespace {
template <int D>
void set_kernels(RowsPlan* pl) {
  using C = rk::RCfg<D>;
  pl->kernel[0] = (const void*)rk::rows_kernel<D, false>;
  pl->kernel[1] = (const void*)rk::rows_kernel<D, true>;
  pl->p0q = C::P0Q;
  pl->p0f = C::P0F;
  pl->p1 = C::P1;
}
// Region layout after the head: P1, XN, O, P0 (each 256-byte aligned).
struct Layout {
  size_t p1, xn, o, p0, total;  // byte offsets from the state's start
};
Layout layout(const RowsPlan* p, bool fresh) {
  const size_t row = (size_t)rk::MR * p->d * 4;
  Layout y;
  y.p1 = kHead;
  y.xn = y.p1 + align_up(p->p1 * 4);
  y.o = y.xn + align_up(row * (fresh ? 2 * p->L + 1 : 1));
  y.p0 = y.o + align_up(row * (fresh ? p->L : 1));
  y.total = y.p0 + align_up((fresh ? (p->p0q + p->p0f) * p->L : std::max(p->p0q, p->p0f)) * 4);
  return y;
}
}  // namespace

RowsPlan* rows_plan_create(const PersistentWeights& w, int cus) {
  const int d = (int)w.cfg.n_embd, H = (int)w.cfg.n_head;
  if (w.wtype != W_F32 || cus < rk::G || H * rk::HD != d || w.cfg.n_layer == 0) return nullptr;
  RowsPlan* pl = new RowsPlan();
  if (d == 128) {
    set_kernels<128>(pl);
  } else if (d == 768) {
    set_kernels<768>(pl);
  } else if (d == 1024) {
    set_kernels<1024>(pl);
  } else {
    delete pl;
    return nullptr;
  }
  pl->d = d;
  pl->H = H;
  pl->V = (int)w.cfg.vocab_size;
  pl->L = (int)w.cfg.n_layer;
  pl->P = (int)w.cfg.n_positions;
  std::vector<rk::RLayer> lay(pl->L);
  for (int l = 0; l < pl->L; ++l) {
    const PersistentLayer& s = w.layers[l];
    lay[l] = {static_cast<const float*>(s.wqkv), static_cast<const float*>(s.waproj),
              static_cast<const float*>(s.wfc), static_cast<const float*>(s.wmproj), s.bqkv, s.baproj, s.bfc,
              s.bmproj, s.ln1w, s.ln1b, s.ln2w, s.ln2b};
  }
  if (hipMalloc(&pl->layers_dev, sizeof(rk::RLayer) * pl->L) != hipSuccess ||
      hipMemcpy(pl->layers_dev, lay.data(), sizeof(rk::RLayer) * pl->L, hipMemcpyHostToDevice) != hipSuccess) {
    rows_plan_destroy(pl);
    return nullptr;
  }
  rk::RParams& b = pl->base;
  b.layers = pl->layers_dev;
  b.wte = static_cast<const float*>(w.wte);
  b.wpe = w.wpe;
  b.lnfw = w.lnfw;
  b.lnfb = w.lnfb;
  b.L = pl->L;
  b.P = pl->P;
  b.V = pl->V;
  b.eps = w.cfg.layer_norm_epsilon;
  return pl;
}

void rows_plan_destroy(RowsPlan* p) {
  if (!p) return;
  if (p->layers_dev) (void)hipFree(p->layers_dev);
  delete p;
}

bool rows_supported(const RowsPlan* p, int S, int T) {
  return p && S >= 1 && T >= 1 && S <= rk::SMAX && T <= rk::TMAX && S * T <= rk::MR;
}

size_t rows_state_bytes(const RowsPlan* p, bool fresh) { return layout(p, fresh).total; }

namespace {
// Head layout: flags [G][FS] u64 (32 KiB), then epoch (u64), done, err.
rk::u64* head_flags(void* mem) { return static_cast<rk::u64*>(mem); }
rk::u64* head_epoch(void* mem) { return reinterpret_cast<rk::u64*>(static_cast<char*>(mem) + 32768); }
unsigned* head_done(void* mem) { return reinterpret_cast<unsigned*>(static_cast<char*>(mem) + 32768 + 256); }
unsigned* head_err(void* mem) { return reinterpret_cast<unsigned*>(static_cast<char*>(mem) + 32768 + 512); }
}  // namespace

RowsState* rows_state_create(const RowsPlan* p) {
  void* mem = nullptr;
  if (hipMalloc(&mem, rows_state_bytes(p, true)) != hipSuccess) return nullptr;
  const rk::u64 one = 1;
  if (hipMemset(mem, 0, kHead) != hipSuccess ||
      hipMemcpy(head_epoch(mem), &one, sizeof(one), hipMemcpyHostToDevice) != hipSuccess) {
    (void)hipFree(mem);
    return nullptr;
  }
  RowsState* s = new RowsState();
  s->mem = mem;
  s->owned = true;
  s->fresh = true;
  return s;
}

void rows_state_destroy(RowsState* s) {
  if (!s) return;
  if (s->owned && s->mem) (void)hipFree(s->mem);
  delete s;
}

unsigned* rows_err(RowsState* s) { return head_err(s->mem); }

namespace {
rk::u64* trace_buf() {
  static rk::u64* buf = nullptr;
  static bool tried = false;
  if (!tried) {
    tried = true;
    const char* f = getenv("RTG_ROWS_TRACE");
    if (f && f[0] && hipMalloc(&buf, (size_t)rk::G * rk::TRACE_WORDS * 8) != hipSuccess) buf = nullptr;
  }
  return buf;
}
}  // namespace

hipError_t rows_forward(const RowsPlan* p, RowsState* s, hipStream_t stream, float* kc, float* vc, long kv_layer,
                        const uint32_t* ids_dev, int S, int T, int past, const int* pos_dev, float* logits,
                        const RowsFinish* fin, uint64_t* trace) {
  if (!rows_supported(p, S, T)) return hipErrorInvalidValue;
  rk::RParams a = p->base;
  a.kc = kc;
  a.vc = vc;
  a.kv_layer = kv_layer;
  a.M = S * T;
  a.S = S;
  a.T = T;
  a.past = past;
  a.pos_dev = pos_dev;
  a.ids = ids_dev;
  const Layout y = layout(p, s->fresh);
  char* base = static_cast<char*>(s->mem);
  const long row = (long)rk::MR * p->d;
  a.p1 = reinterpret_cast<float*>(base + y.p1);
  a.xn = reinterpret_cast<float*>(base + y.xn);
  a.xn_stride = s->fresh ? row : 0;
  a.o = reinterpret_cast<float*>(base + y.o);
  a.o_stride = s->fresh ? row : 0;
  a.p0 = reinterpret_cast<float*>(base + y.p0);
  a.p0_stride = s->fresh ? (long)(p->p0q + p->p0f) : 0;
  a.p0_fc = s->fresh ? (long)p->p0q : 0;
  a.logits = logits;
  if (fin) {
    a.keys = fin->keys;
    a.lm_last = S <= rk::LM_LAST_MAX;
    a.token = fin->token;
    a.ids_out = fin->ids_out;
    a.ld_ids = fin->ld_ids;
    a.fin_pos = fin->pos;
    a.step = fin->step;
  }
  a.flags = head_flags(s->mem);
  a.epoch = head_epoch(s->mem);
  a.done = head_done(s->mem);
  a.err = head_err(s->mem);
  a.trace = trace ? reinterpret_cast<rk::u64*>(trace) : trace_buf();
  // test hook RTG_TEST_ROWS_WAIT=<wait code>: that wait times out (the
  // host then reports the error)
  a.force_wait = 0;
  if (const char* t = getenv("RTG_TEST_ROWS_WAIT")) a.force_wait = (unsigned)strtoul(t, nullptr, 10);
  void* args[] = {&a};
  return hipLaunchKernel(p->kernel[s->fresh ? 1 : 0], dim3(rk::G), dim3(rk::NTH), args, 0, stream);
}

void rows_dump_trace() {
  rk::u64* buf = trace_buf();
  const char* f = getenv("RTG_ROWS_TRACE");
  if (!buf || !f) return;
  std::vector<rk::u64> h((size_t)rk::G * rk::TRACE_WORDS);
  if (hipMemcpy(h.data(), buf, h.size() * 8, hipMemcpyDeviceToHost) != hipSuccess) return;
  if (FILE* fp = fopen(f, "wb")) {
    fwrite(h.data(), 8, h.size(), fp);
    fclose(fp);
  }
}

}  // namespace rtg
