// Host side of the persistent decode step (see decode_persistent_kernel.h):
// plan (model geometry checks, per-layer pointer table), per-cache state
// (tagged exchange buffers, epoch, error flag) and the launch.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <mutex>
#include <vector>

#include "decode_persistent.h"
#include "decode_persistent_kernel.h"
#include "decode_tile.h"

namespace rtg {
namespace pk {
// Kernel instances, one per (width, largest vocabulary, weight storage);
// defined in the decode_persistent_inst_*.hip files. A model whose vocabulary
// is at most an instance's runs on it (the LM head's rows then go to fewer
// workgroups).
const void* kernel_128_512_f32();
const void* kernel_128_512_bf16();
const void* kernel_768_50257_f32();
const void* kernel_768_50257_bf16();
const void* kernel_1024_50257_f32();
const void* kernel_1024_50257_bf16();
const void* kernel_1280_50257_f32();
const void* kernel_1600_50257_bf16();
}  // namespace pk

// LayerNorm folded into the GEMV that follows it: for output row r of
// W^T[N][K] (row r contiguous), s[r] = sum_k W[r][k] g[k] and
// c[r] = bias[r] + sum_k W[r][k] b[k], accumulated in double. One wave per row.
__global__ void ln_fold_kernel(const void* W, int wtype, int N, int K, const float* g, const float* b,
                               const float* bias, float* s, float* c) {
  const int r = blockIdx.x * (blockDim.x / 64) + (int)(threadIdx.x / 64);
  const int lane = threadIdx.x & 63;
  if (r >= N) return;
  double ss = 0.0, cc = 0.0;
  for (int k = lane; k < K; k += 64) {
    const float w = wtype == W_F32 ? static_cast<const float*>(W)[(long)r * K + k]
                                   : __uint_as_float((uint32_t)static_cast<const uint16_t*>(W)[(long)r * K + k] << 16);
    ss += (double)w * (double)g[k];
    cc += (double)w * (double)b[k];
  }
  for (int o = 32; o > 0; o >>= 1) {
    ss += __shfl_xor(ss, o, 64);
    cc += __shfl_xor(cc, o, 64);
  }
  if (lane == 0) {
    s[r] = (float)ss;
    c[r] = (float)((bias ? (double)bias[r] : 0.0) + cc);
  }
}

bool ln_fold(const void* W, int wtype, int N, int K, const float* g, const float* b, const float* bias, float* s,
             float* c) {
  hipLaunchKernelGGL(ln_fold_kernel, dim3((N + 3) / 4), dim3(256), 0, 0, W, wtype, N, K, g, b, bias, s, c);
  return hipGetLastError() == hipSuccess;
}

namespace {
struct Inst {
  int d, v, wtype;
  const void* (*fn)();
};
const Inst kInstances[] = {
    {128, 512, W_F32, pk::kernel_128_512_f32},       {128, 512, W_BF16, pk::kernel_128_512_bf16},
    {768, 50257, W_F32, pk::kernel_768_50257_f32},   {768, 50257, W_BF16, pk::kernel_768_50257_bf16},
    {1024, 50257, W_F32, pk::kernel_1024_50257_f32}, {1024, 50257, W_BF16, pk::kernel_1024_50257_bf16},
    {1280, 50257, W_F32, pk::kernel_1280_50257_f32}, {1600, 50257, W_BF16, pk::kernel_1600_50257_bf16},
};
}  // namespace

struct PersistentPlan {
  PersistentWeights w;
  const void* kernel = nullptr;  // null: shape not supported, the graph path runs
  pk::Params base{};
  pk::LayerPtrs* layers_dev = nullptr;
  void* zeros = nullptr;
  float* fold = nullptr;  // folded LayerNorm constants (LayerPtrs::sq etc., Params::sl/cl)
  TilePlan* tile = nullptr;  // the tiled step (decode_tile_kernel.h) for short contexts, where built
};

struct PersistentState {
  PersistentPlan* plan;
  pk::Params p;
  tk::TParams tp{};  // the tiled step's parameters (same decode state, its own exchange words)
  pk::u64* ttags = nullptr;
  pk::u64* tags = nullptr;
  unsigned* epoch = nullptr;
  unsigned* err = nullptr;
  pk::u64* trace = nullptr;
  unsigned* done = nullptr;
};

PersistentPlan* persistent_plan_create(const PersistentWeights& w) {
  PersistentPlan* pl = new PersistentPlan();
  pl->w = w;
  const int d = (int)w.cfg.n_embd, H = (int)w.cfg.n_head, V = (int)w.cfg.vocab_size, L = (int)w.cfg.n_layer;
  const int P = (int)w.cfg.n_positions;
  int dev = 0, cus = 0;
  hipGetDevice(&dev);
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < pk::G)
    return pl;
  if (H <= 0 || d != H * pk::HD || L <= 0 || P <= 0) return pl;
  const void* fn = nullptr;
  for (const Inst& in : kInstances)
    if (in.d == d && V >= 1 && V <= in.v && in.wtype == w.wtype) fn = in.fn();
  if (!fn) return pl;
  // folded constants: per layer sq, cq [3d] and sf, cf [4d]; then sl, cl [V]
  const size_t per_layer = 2 * (size_t)(3 * d) + 2 * (size_t)(4 * d);
  const size_t fold_floats = per_layer * L + 2 * (size_t)V;
  if (hipDeviceSynchronize() != hipSuccess || hipMalloc(&pl->fold, fold_floats * 4) != hipSuccess) return pl;
  std::vector<pk::LayerPtrs> lp(L);
  for (int i = 0; i < L; ++i) {
    const PersistentLayer& s = w.layers[i];
    float* f = pl->fold + per_layer * i;
    float *sq = f, *cq = f + 3 * d, *sf = f + 6 * d, *cf = f + 10 * d;
    if (!ln_fold(s.wqkv, w.wtype, 3 * d, d, s.ln1w, s.ln1b, s.bqkv, sq, cq) ||
        !ln_fold(s.wfc, w.wtype, 4 * d, d, s.ln2w, s.ln2b, s.bfc, sf, cf))
      return pl;
    lp[i] = {s.wqkv, s.waproj, s.wfc, s.wmproj, s.bqkv, s.baproj, s.bfc, s.bmproj, s.ln1w, s.ln1b, s.ln2w, s.ln2b,
             sq, cq, sf, cf};
  }
  float* sl = pl->fold + per_layer * L;
  float* cl = sl + V;
  if (!ln_fold(w.wte, w.wtype, V, d, w.lnfw, w.lnfb, nullptr, sl, cl) || hipDeviceSynchronize() != hipSuccess)
    return pl;
  if (hipMalloc(&pl->layers_dev, sizeof(pk::LayerPtrs) * L) != hipSuccess) return pl;
  if (hipMemcpy(pl->layers_dev, lp.data(), sizeof(pk::LayerPtrs) * L, hipMemcpyHostToDevice) != hipSuccess)
    return pl;
  if (hipMalloc(&pl->zeros, 4096) != hipSuccess || hipMemset(pl->zeros, 0, 4096) != hipSuccess) return pl;
  pk::Params& p = pl->base;
  p.dummy = pl->zeros;
  p.layers = pl->layers_dev;
  p.wte = w.wte;
  p.wpe = w.wpe;
  p.lnfw = w.lnfw;
  p.lnfb = w.lnfb;
  p.sl = sl;
  p.cl = cl;
  p.L = L;
  p.P = P;
  p.V = V;
  p.eps = w.cfg.layer_norm_epsilon;
  p.kv_layer = (long)H * P * pk::HD;
  // Tagged exchange regions of one layer: one slot of whole 128-byte lines per
  // producer (workgroup rows of a GEMV phase, or one attention item).
  auto region = [](int n) { return pk::G * pk::slot_words((n + pk::G - 1) / pk::G); };
  p.o_qkv = 0;
  p.o_att = region(3 * d);
  p.o_head = p.o_att + pk::MAX_ITEMS * pk::ITEM_SLOT;  // merged outputs of chunked heads
  p.o_x2 = p.o_head + H * pk::ITEM_SLOT;
  p.o_h = p.o_x2 + region(d);
  p.o_x3 = p.o_h + region(4 * d);
  p.lw = p.o_x3 + region(d);
  pl->kernel = fn;
  // The tiled step is opt-in: measured slower than the row-split step at c1
  // (253.6 against 209 us per token), it is kept for its exact block-centred
  // LayerNorm and as the measured alternative exchange structure.
  const char* te = getenv("RTG_TILE_STEP");
  if (tile_supported(d, H, V, w.wtype, cus) && te && te[0] == '1') pl->tile = tile_plan_create(w);
  return pl;
}

void persistent_plan_destroy(PersistentPlan* pl) {
  if (!pl) return;
  if (pl->layers_dev) hipFree(pl->layers_dev);
  if (pl->zeros) hipFree(pl->zeros);
  if (pl->fold) hipFree(pl->fold);
  tile_plan_destroy(pl->tile);
  delete pl;
}

bool persistent_supported(const PersistentPlan* pl, int batch) {
  if (!pl || !pl->kernel || batch != 1) return false;
  const char* off = getenv("RTG_DISABLE_PERSISTENT");
  return !(off && off[0] == '1');
}

PersistentState* persistent_state_create(PersistentPlan* pl, float* kcache, float* vcache, int batch,
                                         uint32_t* token_dev, int* pos_dev, float* logits,
                                         unsigned long long* keys, uint32_t* ids_dev, int* step_dev) {
  if (!persistent_supported(pl, batch)) return nullptr;
  PersistentState* s = new PersistentState();
  s->plan = pl;
  s->p = pl->base;
  pk::Params& p = s->p;
  const size_t words = (size_t)p.lw * p.L;
  if (hipMalloc(&s->tags, words * 8) != hipSuccess || hipMalloc(&s->epoch, 256) != hipSuccess ||
      hipMalloc(&s->err, 256) != hipSuccess || hipMalloc(&s->done, 256) != hipSuccess) {
    persistent_state_destroy(s);
    return nullptr;
  }
  // tag 0 never matches: the epoch starts at 1 and only grows
  if (hipMemset(s->tags, 0, words * 8) != hipSuccess || hipMemset(s->err, 0, 256) != hipSuccess ||
      hipMemset(s->done, 0, 256) != hipSuccess) {
    persistent_state_destroy(s);
    return nullptr;
  }
  const unsigned one = 1;
  if (hipMemcpy(s->epoch, &one, 4, hipMemcpyHostToDevice) != hipSuccess) {
    persistent_state_destroy(s);
    return nullptr;
  }
  p.tag = s->tags;
  p.epoch = s->epoch;
  p.err = s->err;
  p.trace = nullptr;
  if (const char* tf = getenv("RTG_TRACE_FILE")) {
    // per-workgroup phase timestamps of the latest step, written on request
    const size_t tbytes = (size_t)pk::G * pk::TRACE_STRIDE * 8;
    if (tf[0] && hipMalloc(&s->trace, tbytes) == hipSuccess && hipMemset(s->trace, 0, tbytes) == hipSuccess)
      p.trace = s->trace;
  }
  p.kc = kcache;
  p.vc = vcache;
  p.token = token_dev;
  p.pos = pos_dev;
  p.logits = logits;
  p.keys = keys;
  p.ids_out = ids_dev;
  p.step = step_dev;
  p.done = s->done;
  if (const TilePlan* tp = pl->tile) {
    // the tiled step shares the decode state (token, position, epoch, keys,
    // error word) and has its own exchange words; tag 0 never matches
    if (hipMalloc(&s->ttags, tp->tag_words * 8) != hipSuccess ||
        hipMemset(s->ttags, 0, tp->tag_words * 8) != hipSuccess) {
      persistent_state_destroy(s);
      return nullptr;
    }
    tk::TParams& t = s->tp;
    t = tp->base;
    t.kc = kcache;
    t.vc = vcache;
    t.token = token_dev;
    t.pos = pos_dev;
    t.ids_out = ids_dev;
    t.step = step_dev;
    t.done = s->done;
    t.epoch = s->epoch;
    t.tag = s->ttags;
    t.logits = logits;
    t.keys = keys;
    t.err = s->err;
    t.trace = p.trace;
    t.dummy = pl->zeros;
  }
  return s;
}

void persistent_state_destroy(PersistentState* s) {
  if (!s) return;
  if (s->tags) hipFree(s->tags);
  if (s->epoch) hipFree(s->epoch);
  if (s->err) hipFree(s->err);
  if (s->trace) hipFree(s->trace);
  if (s->done) hipFree(s->done);
  if (s->ttags) hipFree(s->ttags);
  delete s;
}

void persistent_dump_trace(PersistentState* s) {
  const char* tf = getenv("RTG_TRACE_FILE");
  if (!s || !s->trace || !tf) return;
  std::vector<pk::u64> h((size_t)pk::G * pk::TRACE_STRIDE);
  if (hipMemcpy(h.data(), s->trace, h.size() * 8, hipMemcpyDeviceToHost) != hipSuccess) return;
  if (FILE* f = fopen(tf, "wb")) {
    const int hdr[4] = {pk::G, pk::TRACE_STRIDE, s->p.L, 0};
    fwrite(hdr, sizeof hdr, 1, f);
    fwrite(h.data(), 8, h.size(), f);
    fclose(f);
  }
}

unsigned* persistent_epoch(PersistentState* s) { return s ? s->epoch : nullptr; }
unsigned* persistent_err(PersistentState* s) { return s ? s->err : nullptr; }

hipError_t persistent_decode_step(PersistentState* s, hipStream_t stream, bool cooperative, int pos) {
  // the tiled step where the plan has one and the context fits its LDS
  // windows; both kernels keep the same decode state, so steps may alternate
  if (s->plan->tile && s->ttags && pos >= 0 && pos + 1 <= tile_max_len())
    return tile_decode_step(s->plan->tile, s->tp, stream, cooperative);
  // test hook RTG_TEST_DECODE_WAIT="<polling rounds>": the step's layer-1
  // input fetch times out after that many rounds (the host reports it)
  s->p.test_spins = 0;
  if (const char* t = getenv("RTG_TEST_DECODE_WAIT")) s->p.test_spins = (unsigned)strtoul(t, nullptr, 10);
  void* args[] = {&s->p};
  const void* fn = s->plan->kernel;
  if (cooperative) return hipLaunchCooperativeKernel(fn, dim3(pk::G), dim3(pk::NTHREADS), args, 0, stream);
  // A plain launch of one workgroup per CU (the kernel's LDS footprint admits
  // no second one per CU). The workgroups wait on each other, so they must all
  // become resident: the caller holds persistent_launch_lock for the device
  // from the first step it enqueues until its stream has drained, so no other
  // persistent step of this process can take part of the CUs meanwhile.
  // Ordinary kernels of other streams finish by themselves and only delay the
  // step; every wait is bounded should residency still fail (another process
  // on the same GPU), and the host then reports an error.
  return hipLaunchKernel(fn, dim3(pk::G), dim3(pk::NTHREADS), args, 0, stream);
}

std::mutex& persistent_launch_lock(int device) {
  static std::mutex locks[64];
  return locks[(unsigned)device % 64u];
}

}  // namespace rtg
