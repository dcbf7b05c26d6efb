// Multi-tensor optimiser kernels: one launch updates up to kMaxT tensors.
//
// The reference dispatches one shader per parameter tensor (SGDBatch loops
// over `sgd` dispatches, engine.cpp:436-485; AdamW.step loops over `adam`
// dispatches from Python, nn_engine.py:2217-2238; SGDBatchClipped runs
// grad_sq_reduce per tensor, grad_norm_final, then sgd_clipped per tensor,
// engine.cpp:494-614).  Here a table of tensor pointers travels as a kernel
// argument and each 256-thread block owns a 4096-element chunk of one tensor;
// float4 traffic, per-element arithmetic identical to the HLSL.
#include "dce_internal.h"

#include <algorithm>
#include <cmath>
#include <vector>

namespace dce {

constexpr int kMaxT = 48;
constexpr uint32_t kChunk = 4096;  // elements per block (256 threads x 16)

struct Table {
  float* w[kMaxT];
  float* g[kMaxT];
  float* m[kMaxT];
  float* v[kMaxT];
  uint32_t n[kMaxT];
  uint32_t start[kMaxT + 1];  // first block of each tensor
  uint32_t count;
};

static inline uint32_t cdiv(uint64_t a, uint64_t b) { return uint32_t((a + b - 1) / b); }

__device__ __forceinline__ int find_tensor(const Table& t, uint32_t blk) {
  int lo = 0, hi = int(t.count) - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (t.start[mid] <= blk) lo = mid; else hi = mid - 1;
  }
  return lo;
}

struct SgdOp {  // nn_sgd.hlsl:7-10
  float lr, clip;
  __device__ void operator()(float& w, float& g, float&, float&) const {
    float gv = g;
    if (gv > clip) gv = clip;
    if (gv < -clip) gv = -clip;
    w = w - lr * gv;
  }
};
struct SgdScaledOp {  // nn_sgd_clipped.hlsl:18-19
  float lr, scale;
  __device__ void operator()(float& w, float& g, float&, float&) const { w -= lr * g * scale; }
};
struct ScaleOp {
  float scale;
  __device__ void operator()(float&, float& g, float&, float&) const { g = g * scale; }
};
struct AdamOp {  // nn_adam.hlsl:20-33
  float step, b1, b2, eps, wd, clip;
  __device__ void operator()(float& w, float& g, float& m, float& v) const {
    float gv = g;
    if (gv > clip) gv = clip;
    if (gv < -clip) gv = -clip;
    const float cw = w;
    const float mt = b1 * m + (1.0f - b1) * gv;
    const float vt = b2 * v + (1.0f - b2) * gv * gv;
    m = mt;
    v = vt;
    w = cw - wd * cw - step * mt / (sqrtf(vt) + eps);
  }
};

// WRITE: bit0 w, bit1 g, bit2 m, bit3 v.  READ likewise.
// NT: streaming (nontemporal) accesses, for a pass larger than the MALL.
template <class Op, int READ, int WRITE, bool NT>
__device__ __forceinline__ void apply_chunk(const Table& t, const Op& op, int ti, uint32_t c0) {
  const uint32_t n = t.n[ti];
  float* w = t.w[ti];
  float* g = t.g[ti];
  float* m = t.m[ti];
  float* v = t.v[ti];
  const uint32_t end = min(n, c0 + kChunk);
  if (c0 + kChunk <= n && ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(g) |
                            reinterpret_cast<uintptr_t>(m) | reinterpret_cast<uintptr_t>(v)) & 15) == 0) {
    // Whole, aligned chunk: every quad of the thread is loaded before any is
    // stored, so all of them are in flight together.
    f4 W[4], G[4], M[4], V[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t i = c0 + (j * 256 + threadIdx.x) * 4;
      W[j] = G[j] = M[j] = V[j] = f4{0.f, 0.f, 0.f, 0.f};
      if (READ & 1) W[j] = ld4s<NT>(w + i);
      if (READ & 2) G[j] = ld4s<NT>(g + i);
      if (READ & 4) M[j] = ld4s<NT>(m + i);
      if (READ & 8) V[j] = ld4s<NT>(v + i);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float a = W[j][e], b = G[j][e], c = M[j][e], d = V[j][e];
        op(a, b, c, d);
        W[j][e] = a;
        G[j][e] = b;
        M[j][e] = c;
        V[j][e] = d;
      }
    }
    // Nontemporal stores only when several streams are written: with one
    // written stream (SGD: 115 -> 110 us over AlexNet's 61 M parameters) the
    // default policy stores faster, with three (Adam: 293 vs 330 us) the
    // streaming one does.
    constexpr bool NTS = NT && (WRITE & (WRITE - 1)) != 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t i = c0 + (j * 256 + threadIdx.x) * 4;
      if (WRITE & 1) st4s<NTS>(w + i, W[j]);
      if (WRITE & 2) st4s<NTS>(g + i, G[j]);
      if (WRITE & 4) st4s<NTS>(m + i, M[j]);
      if (WRITE & 8) st4s<NTS>(v + i, V[j]);
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t i = c0 + (j * 256 + threadIdx.x) * 4;
    if (i + 3 < end) {
      f4 W = {0, 0, 0, 0}, G = W, M = W, V = W;
      if (READ & 1) W = *reinterpret_cast<const f4*>(w + i);
      if (READ & 2) G = *reinterpret_cast<const f4*>(g + i);
      if (READ & 4) M = *reinterpret_cast<const f4*>(m + i);
      if (READ & 8) V = *reinterpret_cast<const f4*>(v + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float a = W[e], b = G[e], c = M[e], d = V[e];
        op(a, b, c, d);
        W[e] = a; G[e] = b; M[e] = c; V[e] = d;
      }
      if (WRITE & 1) *reinterpret_cast<f4*>(w + i) = W;
      if (WRITE & 2) *reinterpret_cast<f4*>(g + i) = G;
      if (WRITE & 4) *reinterpret_cast<f4*>(m + i) = M;
      if (WRITE & 8) *reinterpret_cast<f4*>(v + i) = V;
    } else {
      for (uint32_t k = i; k < end && k < i + 4; ++k) {
        float a = (READ & 1) ? w[k] : 0.f, b = (READ & 2) ? g[k] : 0.f;
        float c = (READ & 4) ? m[k] : 0.f, d = (READ & 8) ? v[k] : 0.f;
        op(a, b, c, d);
        if (WRITE & 1) w[k] = a;
        if (WRITE & 2) g[k] = b;
        if (WRITE & 4) m[k] = c;
        if (WRITE & 8) v[k] = d;
      }
    }
  }
}

template <class Op, int READ, int WRITE, bool NT>
__global__ void __launch_bounds__(256) k_multi(const Table t, const Op op) {
  const int ti = find_tensor(t, blockIdx.x);
  apply_chunk<Op, READ, WRITE, NT>(t, op, ti, (blockIdx.x - t.start[ti]) * kChunk);
}

// Scale read from device memory (norm clip): skipped entirely when 1.
template <class Op, int READ, int WRITE, bool NT>
__global__ void __launch_bounds__(256) k_multi_devscale(const Table t, Op op, const float* ns) {
  const float scale = ns[1];
  if (Op::kSkipUnit && scale == 1.0f) return;
  op.scale = scale;
  const int ti = find_tensor(t, blockIdx.x);
  apply_chunk<Op, READ, WRITE, NT>(t, op, ti, (blockIdx.x - t.start[ti]) * kChunk);
}
// Adam with the bias-corrected step size read from device memory
// (state[1], written by k_adam_tick just before), so that a recorded step
// replays with the step size of its own step count.
template <bool NT>
__global__ void __launch_bounds__(256) k_multi_adam_dev(const Table t, AdamOp op,
                                                          const float* state) {
  op.step = state[1];
  const int ti = find_tensor(t, blockIdx.x);
  apply_chunk<AdamOp, 15, 13, NT>(t, op, ti, (blockIdx.x - t.start[ti]) * kChunk);
}

// Step counter of Adam / AdamW on the device: state[0] holds t (u32 bits),
// state[1] the step size lr*sqrt(1 - b2^t)/(1 - b1^t) for that t.  t_set > 0
// sets the counter (an eager step whose count the host knows) and stores the
// host's step size, evaluated as the reference evaluates it in Python and
// hands the float to the shader (nn_engine.py:2219-2220).  t_set == 0
// advances the counter by one (a recorded step, whose every replay is the
// next step) and evaluates the same expression here, in double from the
// double hyper-parameters, rounded once to float.
__global__ void k_adam_tick(float* state, uint32_t t_set, float step_host, double lr, double b1,
                            double b2) {
  if (threadIdx.x != 0) return;
  const uint32_t t = t_set ? t_set : __float_as_uint(state[0]) + 1u;
  const double td = double(t);
  state[0] = __uint_as_float(t);
  state[1] = t_set ? step_host : float(lr * sqrt(1.0 - pow(b2, td)) / (1.0 - pow(b1, td)));
}

struct SgdScaledDev : SgdScaledOp {
  static constexpr bool kSkipUnit = false;
};
struct ScaleDev : ScaleOp {
  static constexpr bool kSkipUnit = true;
};

// Σ g² per block (double), written at part[base + block].
template <bool NT>
__global__ void __launch_bounds__(256) k_multi_sumsq(const Table t, double* part, uint32_t base) {
  __shared__ double sh[4];
  const int ti = find_tensor(t, blockIdx.x);
  const uint32_t c0 = (blockIdx.x - t.start[ti]) * kChunk;
  const uint32_t n = t.n[ti];
  const float* g = t.g[ti];
  const uint32_t end = min(n, c0 + kChunk);
  float acc = 0.f;
  if (c0 + kChunk <= n && (reinterpret_cast<uintptr_t>(g) & 15) == 0) {
    f4 G[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) G[j] = ld4s<NT>(g + c0 + (j * 256 + threadIdx.x) * 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc += G[j][0] * G[j][0] + G[j][1] * G[j][1] + G[j][2] * G[j][2] + G[j][3] * G[j][3];
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t i = c0 + (j * 256 + threadIdx.x) * 4;
      if (i + 3 < end) {
        const f4 G = *reinterpret_cast<const f4*>(g + i);
        acc += G[0] * G[0] + G[1] * G[1] + G[2] * G[2] + G[3] * G[3];
      } else {
        for (uint32_t k = i; k < end && k < i + 4; ++k) acc += g[k] * g[k];
      }
    }
  }
  const double s = wave_reduce(double(acc));
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) part[base + blockIdx.x] = (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

// norm = sqrt(Σ partials); scale = norm > max ? max/(norm + 1e-6) : 1
// (nn_grad_norm_final.hlsl:31-34).
// One block of 1024 threads; thread t adds partials t, t + 1024, ... in
// rounds of 16 loads issued together (one memory round trip per 16384
// partials: AlexNet's 61 M parameters make about 15,000), then a fixed
// shuffle / LDS tree.
__global__ void __launch_bounds__(1024)
    k_norm_final(const double* part, uint32_t total, float maxNorm, float* ns) {
  __shared__ double sh[16];
  double s = 0;
  for (uint32_t i0 = 0; i0 < total; i0 += 16 * 1024) {
    double v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const uint32_t i = i0 + threadIdx.x + u * 1024;
      v[u] = i < total ? part[i] : 0.0;
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) s += v[u];
  }
  s = wave_reduce(s);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    double tot = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) tot += sh[w];
    const float norm = float(sqrt(tot));
    ns[0] = norm;
    ns[1] = (norm > maxNorm) ? (maxNorm / (norm + 1e-6f)) : 1.0f;
  }
}

// Build tables of at most kMaxT tensors from handle arrays; entries whose
// param/grad (or m/v) handle is NULL or not live are skipped.
static bool build_tables(void** params, void** grads, void** m, void** v, const uint32_t* sizes,
                         uint32_t n, bool needW, std::vector<Table>& out, uint32_t* totalBlocks) {
  out.clear();
  Table cur{};
  uint32_t blocks = 0, all = 0;
  for (uint32_t i = 0; i < n; ++i) {
    if (!grads[i] || (needW && !params[i])) continue;
    Buffer* G = as_buffer(grads[i], "optimizer(grad)");
    Buffer* W = needW ? as_buffer(params[i], "optimizer(param)") : nullptr;
    Buffer* M = m ? as_buffer(m[i], "optimizer(m)") : nullptr;
    Buffer* V = v ? as_buffer(v[i], "optimizer(v)") : nullptr;
    if (!G || (needW && !W) || (m && !M) || (v && !V)) return false;
    uint32_t cnt = std::min(sizes[i], G->count);
    if (W) cnt = std::min(cnt, W->count);
    if (M) cnt = std::min(cnt, M->count);
    if (V) cnt = std::min(cnt, V->count);
    if (!cnt) continue;
    if (cur.count == kMaxT) {
      cur.start[cur.count] = blocks;
      out.push_back(cur);
      cur = Table{};
      blocks = 0;
    }
    const uint32_t k = cur.count++;
    cur.w[k] = W ? W->ptr : nullptr;
    cur.g[k] = G->ptr;
    cur.m[k] = M ? M->ptr : nullptr;
    cur.v[k] = V ? V->ptr : nullptr;
    cur.n[k] = cnt;
    cur.start[k] = blocks;
    blocks += cdiv(cnt, kChunk);
    all += cdiv(cnt, kChunk);
  }
  if (cur.count) {
    cur.start[cur.count] = blocks;
    out.push_back(cur);
  }
  if (totalBlocks) *totalBlocks = all;
  return true;
}

static inline uint32_t table_blocks(const Table& t) { return t.start[t.count]; }

static double table_elems(const std::vector<Table>& tabs) {
  double e = 0;
  for (const Table& t : tabs)
    for (uint32_t i = 0; i < t.count; ++i) e += t.n[i];
  return e;
}



bool sgd_multi(void** params, void** grads, const uint32_t* sizes, uint32_t n, float lr,
               float clip) {
  std::vector<Table> tabs;
  if (!build_tables(params, grads, nullptr, nullptr, sizes, n, true, tabs, nullptr)) return false;
  const double bytes = 12.0 * table_elems(tabs);
  const bool nt = stream_nt(bytes);
  ProfScope prof("sgd", 0, bytes);
  for (const Table& t : tabs) {
    if (nt)
      hipLaunchKernelGGL((k_multi<SgdOp, 3, 1, true>), dim3(table_blocks(t)), dim3(256), 0,
                         stream(), t, SgdOp{lr, clip});
    else
      hipLaunchKernelGGL((k_multi<SgdOp, 3, 1, false>), dim3(table_blocks(t)), dim3(256), 0,
                         stream(), t, SgdOp{lr, clip});
    if (!check_launch("SGDBatch")) return false;
  }
  return true;
}

bool grad_norm_multi(void** grads, const uint32_t* sizes, uint32_t n, float max_norm,
                     float* d_ns) {
  std::vector<Table> tabs;
  uint32_t total = 0;
  if (!build_tables(nullptr, grads, nullptr, nullptr, sizes, n, false, tabs, &total)) return false;
  double* part = reinterpret_cast<double*>(workspace(size_t(std::max<uint32_t>(total, 1)) * 2));
  if (!part) return false;
  const double bytes = 4.0 * table_elems(tabs);
  const bool nt = stream_nt(bytes);
  ProfScope prof("grad_norm", 0, bytes);
  uint32_t base = 0;
  for (const Table& t : tabs) {
    if (nt)
      hipLaunchKernelGGL(k_multi_sumsq<true>, dim3(table_blocks(t)), dim3(256), 0, stream(), t,
                         part, base);
    else
      hipLaunchKernelGGL(k_multi_sumsq<false>, dim3(table_blocks(t)), dim3(256), 0, stream(), t,
                         part, base);
    base += table_blocks(t);
  }
  hipLaunchKernelGGL(k_norm_final, dim3(1), dim3(1024), 0, stream(), part, total, max_norm, d_ns);
  return check_launch("grad_norm");
}

bool sgd_scaled_multi(void** params, void** grads, const uint32_t* sizes, uint32_t n, float lr,
                      const float* d_ns) {
  std::vector<Table> tabs;
  if (!build_tables(params, grads, nullptr, nullptr, sizes, n, true, tabs, nullptr)) return false;
  SgdScaledDev op;
  op.lr = lr;
  op.scale = 1.f;
  const double bytes = 12.0 * table_elems(tabs);
  const bool nt = stream_nt(bytes);
  ProfScope prof("sgd_clipped", 0, bytes);
  for (const Table& t : tabs) {
    if (nt)
      hipLaunchKernelGGL((k_multi_devscale<SgdScaledDev, 3, 1, true>), dim3(table_blocks(t)),
                         dim3(256), 0, stream(), t, op, d_ns);
    else
      hipLaunchKernelGGL((k_multi_devscale<SgdScaledDev, 3, 1, false>), dim3(table_blocks(t)),
                         dim3(256), 0, stream(), t, op, d_ns);
    if (!check_launch("SGDBatchClipped")) return false;
  }
  return true;
}

bool scale_grads_multi(void** grads, const uint32_t* sizes, uint32_t n, const float* d_ns) {
  std::vector<Table> tabs;
  if (!build_tables(nullptr, grads, nullptr, nullptr, sizes, n, false, tabs, nullptr)) return false;
  ScaleDev op;
  op.scale = 1.f;
  const double bytes = 8.0 * table_elems(tabs);
  const bool nt = stream_nt(bytes);
  ProfScope prof("clip_scale", 0, bytes);
  for (const Table& t : tabs) {
    if (nt)
      hipLaunchKernelGGL((k_multi_devscale<ScaleDev, 2, 2, true>), dim3(table_blocks(t)),
                         dim3(256), 0, stream(), t, op, d_ns);
    else
      hipLaunchKernelGGL((k_multi_devscale<ScaleDev, 2, 2, false>), dim3(table_blocks(t)),
                         dim3(256), 0, stream(), t, op, d_ns);
    if (!check_launch("ClipGradNorm")) return false;
  }
  return true;
}

bool adam_multi(void** params, void** grads, void** m, void** v, const uint32_t* sizes, uint32_t n,
                float step, float b1, float b2, float eps, float wd, float clip) {
  std::vector<Table> tabs;
  uint32_t total = 0;
  if (!build_tables(params, grads, m, v, sizes, n, true, tabs, &total)) return false;
  const double bytes = 28.0 * table_elems(tabs);
  const bool nt = stream_nt(bytes);
  ProfScope prof("adam", 0, bytes);
  for (const Table& t : tabs) {
    if (nt)
      hipLaunchKernelGGL((k_multi<AdamOp, 15, 13, true>), dim3(table_blocks(t)), dim3(256), 0,
                         stream(), t, AdamOp{step, b1, b2, eps, wd, clip});
    else
      hipLaunchKernelGGL((k_multi<AdamOp, 15, 13, false>), dim3(table_blocks(t)), dim3(256), 0,
                         stream(), t, AdamOp{step, b1, b2, eps, wd, clip});
    if (!check_launch("AdamBatch")) return false;
  }
  return true;
}

bool adam_counted_multi(void** params, void** grads, void** m, void** v,
                        const uint32_t* sizes, uint32_t n, float* state, uint32_t t_set,
                        float step_host, double lr, double b1, double b2, float eps, float wd,
                        float clip) {
  std::vector<Table> tabs;
  if (!build_tables(params, grads, m, v, sizes, n, true, tabs, nullptr)) return false;
  hipLaunchKernelGGL(k_adam_tick, dim3(1), dim3(64), 0, stream(), state, t_set, step_host, lr,
                     b1, b2);
  if (!check_launch("AdamBatchCounted(tick)")) return false;
  const double bytes = 28.0 * table_elems(tabs);
  const bool nt = stream_nt(bytes);
  ProfScope prof("adam", 0, bytes);
  const AdamOp op{0.f, float(b1), float(b2), eps, wd, clip};
  for (const Table& t : tabs) {
    if (nt)
      hipLaunchKernelGGL(k_multi_adam_dev<true>, dim3(table_blocks(t)), dim3(256), 0, stream(), t,
                         op, state);
    else
      hipLaunchKernelGGL(k_multi_adam_dev<false>, dim3(table_blocks(t)), dim3(256), 0, stream(),
                         t, op, state);
    if (!check_launch("AdamBatchCounted")) return false;
  }
  return true;
}

// ---------------------------------------------------------------------------
// Norm clip without allocation.  Callers that may not allocate device memory
// (code under HIP graph capture, tight serving loops) get the kernels of
// ClipGradNorm with their scratch -- the per-block partial sums and the
// [norm, scale] pair -- in this file-scope array instead of the growable
// workspace.  kNoAllocParts partials cover up to kNoAllocParts * kChunk
// gradient elements (fewer when tensors end inside a chunk).  Each GPU holds
// its own copy of the array, at its own address, until the process ends; the
// host uses only the address hipGetSymbolAddress reports for the current
// device (the array's name is a host-side stand-in, not a device address).
// Every call on a GPU shares that GPU's copy: calls overlapping on one GPU
// would race, which the library's single in-order stream rules out for its
// own calls.  Every partial is written before it is read, and the pair is
// written by the final kernel, so nothing needs clearing between calls.
// ---------------------------------------------------------------------------
constexpr uint32_t kNoAllocParts = 65536;
constexpr uint32_t kNoAllocDoubles = kNoAllocParts + 32;  // partials, then the pair
constexpr int kMaxDevices = 64;
static __device__ __align__(256) double scratch[kNoAllocDoubles];
static double* g_scratchDev[kMaxDevices];

bool noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDevices) {
    set_error("InitEngine: device %d beyond the %d the scratch table holds", device, kMaxDevices);
    return false;
  }
  if (g_scratchDev[device]) return true;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) {
    hipGetLastError();
    set_error("InitEngine: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
    return false;
  }
  g_scratchDev[device] = static_cast<double*>(p);
  return true;
}

float clip_grad_norm_noalloc(int device, void** grads, const uint32_t* sizes, uint32_t n,
                             float max_norm, bool capturing) {
  double* part = (device >= 0 && device < kMaxDevices) ? g_scratchDev[device] : nullptr;
  if (!part) {
    set_error("ClipGradNormNoAlloc: no scratch address for device %d", device);
    return -1.0f;
  }
  float* ns = reinterpret_cast<float*>(part + kNoAllocParts);
  // Pass 1: validate every handle and count the partials, before any launch.
  uint64_t total = 0;
  for (uint32_t i = 0; i < n; ++i) {
    if (!grads[i]) continue;
    Buffer* G = as_buffer(grads[i], "ClipGradNormNoAlloc(grad)");
    if (!G) return -1.0f;
    total += cdiv(std::min(sizes[i], G->count), kChunk);
  }
  if (total > kNoAllocParts) {
    set_error("ClipGradNormNoAlloc: %llu partial sums exceed the %u of the static scratch "
              "(at most %u chunks of %u gradient elements)",
              (unsigned long long)total, kNoAllocParts, kNoAllocParts, kChunk);
    return -1.0f;
  }
  // Pass 2: the Σg² partials, one table of at most kMaxT tensors per launch.
  const bool nt = stream_nt(4.0 * double(total) * kChunk);
  Table t{};
  uint32_t base = 0, blocks = 0;
  auto flush_sumsq = [&]() -> bool {
    if (!t.count) return true;
    t.start[t.count] = blocks;
    if (nt)
      hipLaunchKernelGGL(k_multi_sumsq<true>, dim3(blocks), dim3(256), 0, stream(), t, part, base);
    else
      hipLaunchKernelGGL(k_multi_sumsq<false>, dim3(blocks), dim3(256), 0, stream(), t, part, base);
    base += blocks;
    t = Table{};
    blocks = 0;
    return check_launch("ClipGradNormNoAlloc(sumsq)");
  };
  for (uint32_t i = 0; i < n; ++i) {
    if (!grads[i]) continue;
    Buffer* G = static_cast<Buffer*>(grads[i]);
    const uint32_t cnt = std::min(sizes[i], G->count);
    if (!cnt) continue;
    if (t.count == kMaxT && !flush_sumsq()) return -1.0f;
    t.g[t.count] = G->ptr;
    t.n[t.count] = cnt;
    t.start[t.count] = blocks;
    t.count++;
    blocks += cdiv(cnt, kChunk);
  }
  if (!flush_sumsq()) return -1.0f;
  hipLaunchKernelGGL(k_norm_final, dim3(1), dim3(1024), 0, stream(), part, base, max_norm, ns);
  if (!check_launch("ClipGradNormNoAlloc(final)")) return -1.0f;
  // Pass 3: scale in place when the norm exceeds max_norm (read on the device).
  ScaleDev op;
  op.scale = 1.f;
  t = Table{};
  blocks = 0;
  auto flush_scale = [&]() -> bool {
    if (!t.count) return true;
    t.start[t.count] = blocks;
    if (nt)
      hipLaunchKernelGGL((k_multi_devscale<ScaleDev, 2, 2, true>), dim3(blocks), dim3(256), 0,
                         stream(), t, op, ns);
    else
      hipLaunchKernelGGL((k_multi_devscale<ScaleDev, 2, 2, false>), dim3(blocks), dim3(256), 0,
                         stream(), t, op, ns);
    t = Table{};
    blocks = 0;
    return check_launch("ClipGradNormNoAlloc(scale)");
  };
  for (uint32_t i = 0; i < n; ++i) {
    if (!grads[i]) continue;
    Buffer* G = static_cast<Buffer*>(grads[i]);
    const uint32_t cnt = std::min(sizes[i], G->count);
    if (!cnt) continue;
    if (t.count == kMaxT && !flush_scale()) return -1.0f;
    t.g[t.count] = G->ptr;
    t.n[t.count] = cnt;
    t.start[t.count] = blocks;
    t.count++;
    blocks += cdiv(cnt, kChunk);
  }
  if (!flush_scale()) return -1.0f;
  if (capturing) return std::nanf("");  // the norm exists only when the graph runs
  float h[2] = {0.f, 0.f};
  if (hipMemcpyAsync(h, ns, sizeof(h), hipMemcpyDeviceToHost, stream()) != hipSuccess ||
      hipStreamSynchronize(stream()) != hipSuccess) {
    hipGetLastError();
    set_error("ClipGradNormNoAlloc: reading the norm back failed");
    return -1.0f;
  }
  return h[0];
}

}  // namespace dce
