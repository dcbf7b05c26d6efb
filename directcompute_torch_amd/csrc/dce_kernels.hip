// Memory-bound kernels and the RunShader registry.
//
// Each registry entry takes the reference shader's inputs (t-registers),
// outputs (u-registers) and packed constant buffer, validates them on the
// host, and launches a HIP kernel whose grid is derived from the constants.
// Two flavours per hot op:
//   * fast path: every buffer is at least as large as the constants imply ->
//     unchecked, float4-vectorised where the layout allows;
//   * checked path: D3D11 structured-buffer semantics (reads past a buffer
//     return 0, writes past it are dropped), element by element.
// Reductions are deterministic: per-thread partial sums, a fixed-shape
// wave/LDS tree, and (for long rows) per-piece partials summed in a fixed
// order by a second pass.
#include "dce_internal.h"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace dce {

static inline uint32_t cdiv(uint64_t a, uint64_t b) { return uint32_t((a + b - 1) / b); }

__device__ __forceinline__ float ld(const Buf& b, uint32_t i) { return i < b.n ? b.p[i] : 0.f; }
__device__ __forceinline__ void st(const Buf& b, uint32_t i, float v) {
  if (i < b.n) b.p[i] = v;
}
__device__ __forceinline__ uint32_t gtid() { return blockIdx.x * blockDim.x + threadIdx.x; }


// ===========================================================================
// Generic elementwise kernels: out[i] = F(in0[i], in1[i]).
// ===========================================================================
template <class F>
__global__ void k_ew_checked(F f, Buf out, Buf a, Buf b, uint32_t n) {
  const uint32_t i = gtid();
  if (i < n) st(out, i, f(ld(a, i), ld(b, i)));
}

template <class F, bool NT>
__global__ void k_ew_fast(F f, float* __restrict__ out, const float* __restrict__ a,
                          const float* __restrict__ b, uint32_t n) {
  const uint32_t i4 = gtid() * 4;
  if (i4 + 3 < n) {
    const f4 va = ld4s<NT>(a + i4);
    const f4 vb = b ? ld4s<NT>(b + i4) : f4{0.f, 0.f, 0.f, 0.f};
    f4 r;
    r[0] = f(va[0], vb[0]);
    r[1] = f(va[1], vb[1]);
    r[2] = f(va[2], vb[2]);
    r[3] = f(va[3], vb[3]);
    st4s<NT>(out + i4, r);
  } else {
    for (uint32_t i = i4; i < n; ++i) out[i] = f(a[i], b ? b[i] : 0.f);
  }
}

// Launch an elementwise op over n elements; fast path when every buffer
// covers n.  `b` may be unbound (n == 0) for unary ops.
template <class F>
static bool run_ew(const char* what, F f, Buf out, Buf a, Buf b, uint32_t n, bool unary) {
  if (n == 0) return true;
  const double bytes = (unary ? 8.0 : 12.0) * double(n);
  ProfScope prof(what, 0, bytes);
  const bool fast = out.n >= n && a.n >= n && (unary || b.n >= n) && out.p && a.p &&
                    (unary || b.p);
  if (fast) {
    if (stream_nt(bytes))
      hipLaunchKernelGGL((k_ew_fast<F, true>), dim3(cdiv(cdiv(n, 4), 256)), dim3(256), 0,
                         stream(), f, out.p, a.p, unary ? nullptr : b.p, n);
    else
      hipLaunchKernelGGL((k_ew_fast<F, false>), dim3(cdiv(cdiv(n, 4), 256)), dim3(256), 0,
                         stream(), f, out.p, a.p, unary ? nullptr : b.p, n);
  } else {
    hipLaunchKernelGGL(k_ew_checked<F>, dim3(cdiv(n, 256)), dim3(256), 0, stream(), f, out, a,
                       b, n);
  }
  return check_launch(what);
}

struct OpRelu {
  __device__ float operator()(float a, float) const { return fmaxf(0.f, a); }
};
struct OpReluGrad {  // nn_relu_grad.hlsl:8
  __device__ float operator()(float g, float in) const { return in > 0.f ? g : 0.f; }
};
struct OpRelu6 {  // nn_relu6.hlsl:8-9
  __device__ float operator()(float x, float) const { return fminf(fmaxf(x, 0.f), 6.f); }
};
struct OpRelu6Grad {  // nn_relu6_grad.hlsl:9-10
  __device__ float operator()(float g, float x) const { return (x > 0.f && x < 6.f) ? g : 0.f; }
};
struct OpSigmoid {  // nn_sigmoid.hlsl:12
  __device__ float operator()(float x, float) const { return 1.0f / (1.0f + expf(-x)); }
};
struct OpSigmoidGrad {  // nn_sigmoid_grad.hlsl:12-14
  __device__ float operator()(float dy, float y) const { return dy * y * (1.0f - y); }
};
struct OpLeaky {  // nn_leaky_relu.hlsl:13-14
  float alpha;
  __device__ float operator()(float x, float) const { return x > 0.f ? x : x * alpha; }
};
struct OpLeakyGrad {  // nn_leaky_relu_grad.hlsl:13-16
  float alpha;
  __device__ float operator()(float dy, float x) const { return dy * (x > 0.f ? 1.0f : alpha); }
};
struct OpAdd {
  __device__ float operator()(float a, float b) const { return a + b; }
};
struct OpScaleAdd {  // nn_scale_add.hlsl:9
  float alpha, beta;
  __device__ float operator()(float a, float b) const { return alpha * a + beta * b; }
};
struct OpCopy {
  __device__ float operator()(float a, float) const { return a; }
};

__global__ void k_fill(float* __restrict__ p, float v, size_t n) {
  size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (; i < n; i += stride) p[i] = v;
}

bool fill_zero(float* p, size_t n) {
  if (n == 0) return true;
  uint32_t blocks = uint32_t(std::min<size_t>(cdiv(n, 256), size_t(num_cus()) * 16));
  hipLaunchKernelGGL(k_fill, dim3(blocks), dim3(256), 0, stream(), p, 0.f, n);
  return check_launch("fill");
}

// ===========================================================================
// Registry helpers
// ===========================================================================
static Buf bind(void** arr, uint32_t count, uint32_t i) {
  if (!arr || i >= count || !arr[i]) return Buf{nullptr, 0};
  Buffer* b = static_cast<Buffer*>(arr[i]);
  if (b->magic != kMagicLive) {
    set_error("RunShader: slot %u holds a handle that is not live", i);
    return Buf{nullptr, 0};
  }
  return Buf{b->ptr, b->count};
}
static inline Buf S(const Dispatch& d, uint32_t i) { return bind(d.srvs, d.nS, i); }
static inline Buf U(const Dispatch& d, uint32_t i) { return bind(d.uavs, d.nU, i); }
static inline uint32_t CU(const Dispatch& d, uint32_t i) {
  if (!d.cb || (i + 1) * 4 > d.cbBytes) return 0;
  uint32_t v;
  memcpy(&v, d.cb + 4 * i, 4);
  return v;
}
static inline float CF(const Dispatch& d, uint32_t i) {
  uint32_t u = CU(d, i);
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline bool covers(const Buf& b, uint64_t n) { return b.p && uint64_t(b.n) >= n; }

// ===========================================================================
// Elementwise shaders
// ===========================================================================
// relu / relu6 over a batch norm's output whose forward already stored the
// activation (same functor, same elements) adopt that buffer as the output.
static bool sh_relu(const Dispatch& d) {  // nn_relu.hlsl: no constants, bounded by the output
  Buf o = U(d, 0);
  if (d.nS && d.nU && bn_act_adopt(d.srvs[0], d.uavs[0], 1, o.n)) return true;
  return run_ew("relu", OpRelu{}, o, S(d, 0), Buf{nullptr, 0}, o.n, true);
}
static bool sh_relu6(const Dispatch& d) {
  if (d.nS && d.nU && bn_act_adopt(d.srvs[0], d.uavs[0], 2, CU(d, 0))) return true;
  return run_ew("relu6", OpRelu6{}, U(d, 0), S(d, 0), Buf{nullptr, 0}, CU(d, 0), true);
}
static bool sh_sigmoid(const Dispatch& d) {
  return run_ew("sigmoid", OpSigmoid{}, U(d, 0), S(d, 0), Buf{nullptr, 0}, CU(d, 0), true);
}
static bool sh_sigmoid_grad(const Dispatch& d) {
  return run_ew("sigmoid_grad", OpSigmoidGrad{}, U(d, 0), S(d, 0), S(d, 1), CU(d, 0), false);
}
static bool sh_leaky(const Dispatch& d) {
  return run_ew("leaky_relu", OpLeaky{CF(d, 1)}, U(d, 0), S(d, 0), Buf{nullptr, 0}, CU(d, 0),
                true);
}
static bool sh_leaky_grad(const Dispatch& d) {
  return run_ew("leaky_relu_grad", OpLeakyGrad{CF(d, 1)}, U(d, 0), S(d, 0), S(d, 1), CU(d, 0),
                false);
}
static bool sh_add(const Dispatch& d) {  // nn_add.hlsl: count = M*N
  uint64_t n = uint64_t(CU(d, 0)) * CU(d, 1);
  return run_ew("add", OpAdd{}, U(d, 0), S(d, 0), S(d, 1), uint32_t(std::min<uint64_t>(n, 0xFFFFFFFFu)), false);
}
static bool sh_scale_add(const Dispatch& d) {
  return run_ew("scale_add", OpScaleAdd{CF(d, 1), CF(d, 2)}, U(d, 0), S(d, 0), S(d, 1), CU(d, 0),
                false);
}
static bool sh_grad_accum(const Dispatch& d) {  // acc[i] += g[i]
  Buf acc = U(d, 0);
  return run_ew("grad_accum", OpAdd{}, acc, acc, S(d, 0), CU(d, 0), false);
}

// add_bias / bias_relu: C[i] = A[i] + B[i % N] (+ ReLU), i < M*N.
template <bool RELU>
__global__ void k_add_bias(Buf C, Buf A, Buf B, uint32_t n, uint32_t N) {
  const uint32_t i = gtid();
  if (i >= n) return;
  float v = ld(A, i) + ld(B, i % N);
  st(C, i, RELU ? fmaxf(0.f, v) : v);
}
template <bool RELU>
static bool sh_add_bias_t(const Dispatch& d) {
  uint64_t n = uint64_t(CU(d, 0)) * CU(d, 1);
  uint32_t N = CU(d, 1);
  if (!n || !N) return true;
  hipLaunchKernelGGL(k_add_bias<RELU>, dim3(cdiv(n, 256)), dim3(256), 0, stream(), U(d, 0),
                     S(d, 0), S(d, 1), uint32_t(n), N);
  return check_launch("add_bias");
}

// ===========================================================================
// bias_grad: g[c] = sum_{i<rows} G[i*stride_i + c*stride_id]
// (nn_bias_grad.hlsl).  Two layouts matter: stride_id == 1 (columns of a
// row-major matrix: one thread per column, coalesced over columns) and
// stride_i == 1 (contiguous rows: one block per class).
// ===========================================================================
// Block of 1024 = 64 columns x 16 row slices: lane l takes column
// 64*block + l, wave w rows w, w+16, ...; the 16 slice sums of a column are
// then added in slice order.
__global__ void __launch_bounds__(1024)
    k_bias_grad_cols(Buf G, Buf g, uint32_t rows, uint32_t classes, uint32_t si, uint32_t sid) {
  __shared__ float sh[16][64];
  const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t c = blockIdx.x * 64 + lane;
  float s = 0.f;
  if (c < classes) {
#pragma unroll 8
    for (uint32_t i = w; i < rows; i += 16) s += ld(G, i * si + c * sid);
  }
  sh[w][lane] = s;
  __syncthreads();
  if (w == 0 && c < classes) {
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) t += sh[k][lane];
    st(g, c, t);
  }
}
__global__ void k_bias_grad_rows(Buf G, Buf g, uint32_t rows, uint32_t si, uint32_t sid) {
  __shared__ double sh[4];
  const uint32_t c = blockIdx.x;
  float s = 0.f;
  for (uint32_t i = threadIdx.x; i < rows; i += 256) s += ld(G, i * si + c * sid);
  double t = block_sum256(double(s), sh);
  if (threadIdx.x == 0) st(g, c, float(t));
}
static bool sh_bias_grad(const Dispatch& d) {
  uint32_t rows = CU(d, 0), classes = CU(d, 1), si = CU(d, 2), sid = CU(d, 3);
  if (!classes) return true;
  ProfScope prof("bias_grad", 0, 4.0 * double(rows) * classes);
  if (rows >= 4096 && sid != 1) {
    hipLaunchKernelGGL(k_bias_grad_rows, dim3(classes), dim3(256), 0, stream(), S(d, 0), U(d, 0),
                       rows, si, sid);
  } else {
    hipLaunchKernelGGL(k_bias_grad_cols, dim3(cdiv(classes, 64)), dim3(1024), 0, stream(),
                       S(d, 0), U(d, 0), rows, classes, si, sid);
  }
  return check_launch("bias_grad");
}

// ===========================================================================
// Softmax, cross-entropy, its gradient, metrics
// ===========================================================================
// One wave per row: softmax (nn_softmax.hlsl) and/or the row's CE term
// (nn_loss.hlsl:20-32).  The row term goes to rowLoss when non-null.
__global__ void k_softmax_rows(Buf in, Buf out, Buf labels, float* rowLoss, uint32_t B,
                               uint32_t K, int writeSoftmax) {
  const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= B) return;
  const uint32_t base = row * K;
  float mx = -1e30f;
  for (uint32_t j = lane; j < K; j += 64) mx = fmaxf(mx, ld(in, base + j));
  mx = wave_reduce(mx, OpMaxR());
  float s = 0.f;
  for (uint32_t j = lane; j < K; j += 64) s += expf(ld(in, base + j) - mx);
  s = wave_reduce(s);
  if (writeSoftmax) {
    for (uint32_t j = lane; j < K; j += 64) st(out, base + j, expf(ld(in, base + j) - mx) / s);
  }
  if (rowLoss && lane == 0) {
    const uint32_t label = uint32_t(ld(labels, row));
    rowLoss[row] = -(ld(in, base + label) - mx - logf(s));
  }
}
// Rows of at most 64 * NV elements: each lane loads its NV values once (all
// loads in flight together), then the same max, sum (in the same order) and
// outputs as k_softmax_rows, so the results are identical.
template <int NV>
__global__ void k_softmax_rows_reg(Buf in, Buf out, Buf labels, float* rowLoss, uint32_t B,
                                   uint32_t K, int writeSoftmax) {
  const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= B) return;
  const uint32_t base = row * K;
  float v[NV];
#pragma unroll
  for (int u = 0; u < NV; ++u) {
    const uint32_t j = lane + 64 * u;
    v[u] = j < K ? ld(in, base + j) : -1e30f;
  }
  float mx = -1e30f;
#pragma unroll
  for (int u = 0; u < NV; ++u)
    if (lane + 64 * u < K) mx = fmaxf(mx, v[u]);
  mx = wave_reduce(mx, OpMaxR());
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < NV; ++u)
    if (lane + 64 * u < K) s += expf(v[u] - mx);
  s = wave_reduce(s);
  if (writeSoftmax) {
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const uint32_t j = lane + 64 * u;
      if (j < K) st(out, base + j, expf(v[u] - mx) / s);
    }
  }
  if (rowLoss && lane == 0) {
    const uint32_t label = uint32_t(ld(labels, row));
    rowLoss[row] = -(ld(in, base + label) - mx - logf(s));
  }
}
// Launch the register form for rows of up to 1024 elements.
static void softmax_rows(Buf in, Buf out, Buf labels, float* rowLoss, uint32_t B, uint32_t K,
                         int writeSoftmax) {
  const dim3 grid(cdiv(B, 4)), blk(256);
  if (K <= 256)
    hipLaunchKernelGGL(k_softmax_rows_reg<4>, grid, blk, 0, stream(), in, out, labels, rowLoss,
                       B, K, writeSoftmax);
  else if (K <= 1024)
    hipLaunchKernelGGL(k_softmax_rows_reg<16>, grid, blk, 0, stream(), in, out, labels, rowLoss,
                       B, K, writeSoftmax);
  else
    hipLaunchKernelGGL(k_softmax_rows, grid, blk, 0, stream(), in, out, labels, rowLoss, B, K,
                       writeSoftmax);
}
__global__ void k_mean_rows(const float* rowLoss, Buf loss, uint32_t B) {
  __shared__ double sh[4];
  double s = 0;
  for (uint32_t i = threadIdx.x; i < B; i += 256) s += rowLoss[i];
  s = block_sum256(s, sh);
  if (threadIdx.x == 0) st(loss, 0, float(s / double(B)));
}
static bool sh_softmax(const Dispatch& d) {
  uint32_t B = CU(d, 0), K = CU(d, 1);
  if (!B || !K) return true;
  softmax_rows(S(d, 0), U(d, 0), Buf{nullptr, 0}, nullptr, B, K, 1);
  return check_launch("softmax");
}
static bool sh_loss(const Dispatch& d) {
  uint32_t B = CU(d, 0), K = CU(d, 1);
  if (!B || !K) return true;
  float* rl = workspace(B);
  if (!rl) return false;
  softmax_rows(S(d, 0), Buf{nullptr, 0}, S(d, 1), rl, B, K, 0);
  hipLaunchKernelGGL(k_mean_rows, dim3(1), dim3(256), 0, stream(), rl, U(d, 0), B);
  return check_launch("loss");
}
// (p - onehot(label))/B with the one-hot test labels[b] == (float)j.
__global__ void k_softmax_ce_grad(Buf p, Buf labels, Buf g, uint32_t B, uint32_t K) {
  const uint32_t i = gtid();
  if (i >= B * K) return;
  const uint32_t b = i / K, j = i - b * K;
  const float lab = (ld(labels, b) == float(j)) ? 1.0f : 0.0f;
  st(g, i, (ld(p, i) - lab) / float(B));
}
static bool sh_softmax_ce_grad(const Dispatch& d) {
  uint32_t B = CU(d, 0), K = CU(d, 1);
  if (!B || !K) return true;
  hipLaunchKernelGGL(k_softmax_ce_grad, dim3(cdiv(uint64_t(B) * K, 256)), dim3(256), 0, stream(),
                     S(d, 0), S(d, 1), U(d, 0), B, K);
  return check_launch("softmax_ce_grad");
}
// First-max-wins argmax (strict >, from column 0), count matches on a u32 view.
__global__ void k_argmax_correct(Buf logits, Buf labels, Buf cnt, uint32_t B, uint32_t K) {
  const uint32_t i = gtid();
  if (i >= B) return;
  const uint32_t label = uint32_t(ld(labels, i));
  float mx = ld(logits, i * K);
  uint32_t mi = 0;
  for (uint32_t j = 1; j < K; ++j) {
    const float v = ld(logits, i * K + j);
    if (v > mx) {
      mx = v;
      mi = j;
    }
  }
  if (mi == label && cnt.n > 0) atomicAdd(reinterpret_cast<unsigned int*>(cnt.p), 1u);
}
static bool sh_argmax_correct(const Dispatch& d) {
  uint32_t B = CU(d, 0), K = CU(d, 1);
  if (!B || !K) return true;
  hipLaunchKernelGGL(k_argmax_correct, dim3(cdiv(B, 256)), dim3(256), 0, stream(), S(d, 0),
                     S(d, 1), U(d, 0), B, K);
  return check_launch("argmax_correct");
}
__global__ void k_accumulate_scalar(Buf src, Buf dst) {
  if (threadIdx.x == 0 && dst.n > 0) dst.p[0] = dst.p[0] + ld(src, 0);
}
static bool sh_accumulate_scalar(const Dispatch& d) {
  hipLaunchKernelGGL(k_accumulate_scalar, dim3(1), dim3(64), 0, stream(), S(d, 0), U(d, 0));
  return check_launch("accumulate_scalar");
}

// ===========================================================================
// Dice loss (per-sample sums over `size` elements)
// ===========================================================================
// mode 0: Out[b] = 1 - 2I/(P+T+1e-6); mode 1: Sums[b*3 + {0,1,2}] = {I, P, T}
__global__ void k_dice_sums(Buf pred, Buf tgt, Buf out, uint32_t B, uint32_t size, int mode) {
  __shared__ double sh[4];
  const uint32_t b = blockIdx.x;
  float si = 0.f, sp = 0.f, stt = 0.f;
  const uint32_t off = b * size;
  for (uint32_t i = threadIdx.x; i < size; i += 256) {
    const float p = ld(pred, off + i), t = ld(tgt, off + i);
    si += p * t;
    sp += p;
    stt += t;
  }
  const double I = block_sum256(si, sh);
  const double P = block_sum256(sp, sh);
  const double T = block_sum256(stt, sh);
  if (threadIdx.x == 0) {
    if (mode == 0) {
      const float dice = (2.0f * float(I)) / (float(P) + float(T) + 1e-6f);
      st(out, b, 1.0f - dice);
    } else {
      st(out, b * 3 + 0, float(I));
      st(out, b * 3 + 1, float(P));
      st(out, b * 3 + 2, float(T));
    }
  }
}
// Split form for long rows: block (piece, b) sums a contiguous slice of row b
// (float4 loads, several in flight per thread) into double partials
// part[b][piece][3]; k_dice_final adds a row's pieces in order.
__global__ void __launch_bounds__(256)
    k_dice_part(const float* __restrict__ pred, const float* __restrict__ tgt,
                double* __restrict__ part, uint32_t size4, uint32_t pieces) {
  __shared__ double sh[4];
  const uint32_t b = blockIdx.y, pc = blockIdx.x;
  const uint32_t k0 = uint32_t((uint64_t(size4) * pc) / pieces);
  const uint32_t k1 = uint32_t((uint64_t(size4) * (pc + 1)) / pieces);
  const f4* p4 = reinterpret_cast<const f4*>(pred) + size_t(b) * size4;
  const f4* t4 = reinterpret_cast<const f4*>(tgt) + size_t(b) * size4;
  float si = 0.f, sp = 0.f, stt = 0.f;
  for (uint32_t kb = k0 + threadIdx.x; kb < k1; kb += 1024) {
    f4 pv[4], tv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t k = min(kb + u * 256, k1 - 1);
      pv[u] = p4[k];
      tv[u] = t4[k];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (kb + u * 256 >= k1) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        si += pv[u][e] * tv[u][e];
        sp += pv[u][e];
        stt += tv[u][e];
      }
    }
  }
  const double I = block_sum256(si, sh);
  const double P = block_sum256(sp, sh);
  const double T = block_sum256(stt, sh);
  if (threadIdx.x == 0) {
    double* o = part + (size_t(b) * pieces + pc) * 3;
    o[0] = I;
    o[1] = P;
    o[2] = T;
  }
}
__global__ void k_dice_final(const double* part, uint32_t pieces, uint32_t B, Buf out, int mode) {
  const uint32_t b = gtid();
  if (b >= B) return;
  double I = 0, P = 0, T = 0;
  for (uint32_t q = 0; q < pieces; ++q) {
    const double* o = part + (size_t(b) * pieces + q) * 3;
    I += o[0];
    P += o[1];
    T += o[2];
  }
  if (mode == 0) {
    const float dice = (2.0f * float(I)) / (float(P) + float(T) + 1e-6f);
    st(out, b, 1.0f - dice);
  } else {
    st(out, b * 3 + 0, float(I));
    st(out, b * 3 + 1, float(P));
    st(out, b * 3 + 2, float(T));
  }
}

static bool sh_dice_t(const Dispatch& d, int mode) {
  uint32_t B = CU(d, 0), size = CU(d, 1);
  if (!B) return true;
  const Buf pred = S(d, 0), tgt = S(d, 1);
  const uint64_t total = uint64_t(B) * size;
  if (size % 4 == 0 && size >= 4096 && covers(pred, total) && covers(tgt, total) &&
      ((reinterpret_cast<uintptr_t>(pred.p) | reinterpret_cast<uintptr_t>(tgt.p)) & 15) == 0) {
    const uint32_t want = cdiv(uint32_t(num_cus()) * 4, B);
    const uint32_t pieces = std::max<uint32_t>(1, std::min<uint32_t>(want, size / 4096));
    double* part = reinterpret_cast<double*>(workspace(size_t(B) * pieces * 6));
    if (!part) return false;
    hipLaunchKernelGGL(k_dice_part, dim3(pieces, B), dim3(256), 0, stream(), pred.p, tgt.p, part,
                       size / 4, pieces);
    hipLaunchKernelGGL(k_dice_final, dim3(cdiv(B, 256)), dim3(256), 0, stream(), part, pieces, B,
                       U(d, 0), mode);
    return check_launch("dice");
  }
  hipLaunchKernelGGL(k_dice_sums, dim3(B), dim3(256), 0, stream(), pred, tgt, U(d, 0), B, size,
                     mode);
  return check_launch("dice");
}
static bool sh_dice_loss(const Dispatch& d) { return sh_dice_t(d, 0); }
static bool sh_dice_sums(const Dispatch& d) { return sh_dice_t(d, 1); }
// nn_dice_loss_grad.hlsl:22-33
__global__ void k_dice_grad(Buf pred, Buf tgt, Buf sums, Buf dx, uint32_t B, uint32_t size) {
  const uint32_t i = gtid();
  if (i >= B * size) return;
  const uint32_t b = i / size;
  const float I = ld(sums, b * 3), P = ld(sums, b * 3 + 1), T = ld(sums, b * 3 + 2);
  const float D = P + T + 1e-6f;
  const float t = ld(tgt, i);
  (void)pred;
  const float g = -2.0f * ((t * D) - I) / (D * D);
  st(dx, i, g / float(B));
}
static bool sh_dice_grad(const Dispatch& d) {
  uint32_t B = CU(d, 0), size = CU(d, 1);
  if (!B || !size) return true;
  ProfScope prof("dice_loss_grad", 0, 12.0 * double(B) * size);
  hipLaunchKernelGGL(k_dice_grad, dim3(cdiv(uint64_t(B) * size, 256)), dim3(256), 0, stream(),
                     S(d, 0), S(d, 1), S(d, 2), U(d, 0), B, size);
  return check_launch("dice_grad");
}

// ===========================================================================
// Batch normalisation.  Per-channel sums over N*S elements are split into
// `pieces` contiguous slices of the (n, s) range; slice partials (double)
// are combined in a fixed order by a per-channel finalize.
// ===========================================================================
struct BnPieces {
  uint32_t pieces;
  uint32_t len;  // elements per channel = N*S
};
// Pieces per channel: about eight rounds of resident blocks (8 per CU) over
// all channels, so that the last, partly filled round is a small share of
// the pass; each piece at least 2048 elements long, at most 512 pieces.  At
// 64x96x112x112 (MI355X): backward reduce 92.9 / 88.7 / 87.3 us and
// statistics 55.2 / 54.3 / 69.3 us at 4 / 8 / 16 rounds (beyond 8 the
// statistics' pieces fall under one 1024-quad batch per block).
static BnPieces bn_pieces(uint32_t N, uint32_t C, uint32_t S) {
  BnPieces p;
  p.len = N * S;
  const uint32_t want = cdiv(uint32_t(num_cus()) * 64, std::max<uint32_t>(1, C));
  p.pieces = std::max<uint32_t>(1, std::min<uint32_t>({want, cdiv(p.len, 2048), 512u}));
  return p;
}

// MODE 0: (Σx, Σx²).  MODE 1: (Σdy·x̂, Σdy) with x̂ from mean/var/eps.
template <int MODE, bool CHECK>
__global__ void k_bn_partial(Buf x, Buf dy, Buf mean, Buf var, float eps, uint32_t C, uint32_t S,
                             uint32_t len, uint32_t pieces, FastDiv dS, double* part) {
  __shared__ double sh[4];
  const uint32_t c = blockIdx.y, pc = blockIdx.x;
  const uint32_t i0 = uint32_t((uint64_t(len) * pc) / pieces);
  const uint32_t i1 = uint32_t((uint64_t(len) * (pc + 1)) / pieces);
  float mu = 0.f, rstd = 0.f;
  if (MODE == 1) {
    mu = ld(mean, c);
    rstd = 1.0f / sqrtf(ld(var, c) + eps);
  }
  // Moments accumulate in double: the one-pass variance E[x^2] - E[x]^2
  // cancels catastrophically in float when |mean| >> std.
  double a0 = 0.0, a1 = 0.0;
  for (uint32_t i = i0 + threadIdx.x; i < i1; i += 256) {
    const uint32_t n = fdiv(i, dS);
    const uint32_t idx = n * C * S + c * S + (i - n * S);
    const float xv = CHECK ? ld(x, idx) : x.p[idx];
    if (MODE == 0) {
      a0 += double(xv);
      a1 += double(xv) * double(xv);
    } else {
      const float g = CHECK ? ld(dy, idx) : dy.p[idx];
      const float xh = (xv - mu) * rstd;
      a0 += g * xh;
      a1 += g;
    }
  }
  const double s0 = block_sum256(a0, sh);
  const double s1 = block_sum256(a1, sh);
  if (threadIdx.x == 0) {
    part[(size_t(c) * pieces + pc) * 2 + 0] = s0;
    part[(size_t(c) * pieces + pc) * 2 + 1] = s1;
  }
}

// Same sums over quads when S % 4 == 0 (every quad lies in one plane): the
// piece is a range of quad indices k (plane n = k / (S/4)), read U =
// kBnUnroll quads at a time so that each thread keeps several loads in
// flight (8 measured no faster for the statistics).  The
// grid is (channel, piece) with channels fastest, so the blocks that run
// together read neighbouring planes of the same images (64x96x112x112
// backward reduce 104.6 -> 96.6 us against pieces fastest).
// MODE 2 / 3: dy is not read but made, dy = relu_grad(g, z) / relu6_grad(g,
// z) with the activation shaders' own functors, and stored to dyOut: the
// activation's backward and this reduce in one pass, the same sums in the
// same order as MODE 1 over the stored dy.
constexpr int kBnUnroll = 4;
template <int MODE, bool NT, int U>
__global__ void __launch_bounds__(256)
    k_bn_partial4(const float* __restrict__ x, const float* __restrict__ dy,
                  const float* __restrict__ mean, const float* __restrict__ var, float eps,
                  uint32_t C, uint32_t S4, uint32_t len4, uint32_t pieces, FastDiv dS4,
                  double* __restrict__ part, const float* __restrict__ zin = nullptr,
                  float* __restrict__ dyOut = nullptr) {
  __shared__ double sh[4];
  const uint32_t c = blockIdx.x, pc = blockIdx.y;
  const uint32_t k0 = uint32_t((uint64_t(len4) * pc) / pieces);
  const uint32_t k1 = uint32_t((uint64_t(len4) * (pc + 1)) / pieces);
  float mu = 0.f, rstd = 0.f;
  if (MODE >= 1) {
    mu = mean[c];
    rstd = 1.0f / sqrtf(var[c] + eps);
  }
  double a0 = 0.0, a1 = 0.0;
  // Batches of U quads per thread; the next batch's loads are issued
  // before the current batch is added, so the adds overlap the memory
  // traffic.  Lanes past the piece load quad k0 (in range) and skip it.
  // MODE >= 2: gv holds the incoming gradient and zv the activation input
  // until add() turns them into dy.
  auto load = [&](uint32_t kb, f4 (&xv)[U], f4 (&gv)[U], f4 (&zv)[U], bool (&ok)[U],
                  size_t (&qo)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t k = kb + u * 256;
      ok[u] = k < k1;
      const uint32_t kk = ok[u] ? k : k0;
      const uint32_t n = fdiv(kk, dS4);
      const size_t q = (size_t(n) * C + c) * S4 + (kk - n * S4);
      qo[u] = q;
      xv[u] = ld4s<NT>(x + q * 4);
      if (MODE >= 1) gv[u] = ld4s<NT>(dy + q * 4);
      if (MODE >= 2) zv[u] = ld4s<NT>(zin + q * 4);
    }
  };
  auto add = [&](const f4 (&xv)[U], f4 (&gv)[U], const f4 (&zv)[U], const bool (&ok)[U],
                 const size_t (&qo)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!ok[u]) continue;
      if constexpr (MODE >= 2) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          gv[u][e] = MODE == 2 ? OpReluGrad{}(gv[u][e], zv[u][e]) : OpRelu6Grad{}(gv[u][e], zv[u][e]);
        st4s<NT>(dyOut + qo[u] * 4, gv[u]);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (MODE == 0) {
          a0 += double(xv[u][e]);
          a1 += double(xv[u][e]) * double(xv[u][e]);
        } else {
          const float xh = (xv[u][e] - mu) * rstd;
          a0 += gv[u][e] * xh;
          a1 += gv[u][e];
        }
      }
    }
  };
  f4 xv[U], gv[U], zv[U];
  bool ok[U];
  size_t qo[U];
  uint32_t kb = k0 + threadIdx.x;
  if (kb < k1) load(kb, xv, gv, zv, ok, qo);
  while (kb < k1) {
    const uint32_t kn = kb + 256 * U;
    f4 xn[U], gn[U], zn[U];
    bool okn[U];
    size_t qn[U];
    const bool more = kn < k1;
    if (more) load(kn, xn, gn, zn, okn, qn);
    add(xv, gv, zv, ok, qo);
    if (!more) break;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      xv[u] = xn[u];
      gv[u] = gn[u];
      zv[u] = zn[u];
      ok[u] = okn[u];
      qo[u] = qn[u];
    }
    kb = kn;
  }
  const double s0 = block_sum256(a0, sh);
  const double s1 = block_sum256(a1, sh);
  if (threadIdx.x == 0) {
    part[(size_t(c) * pieces + pc) * 2 + 0] = s0;
    part[(size_t(c) * pieces + pc) * 2 + 1] = s1;
  }
}

// The pieces of channel c summed by one wave: lane l adds pieces l, l+64, ...
// (two moments), then a DPP wave reduction.  Four channels per 256 threads.
__device__ __forceinline__ bool bn_piece_sums(const double* part, uint32_t pieces, uint32_t C,
                                              uint32_t& c, double& s0, double& s1) {
  c = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (c >= C) return false;  // whole waves leave together
  const uint32_t lane = threadIdx.x & 63;
  double a0 = 0, a1 = 0;
  for (uint32_t p = lane; p < pieces; p += 64) {
    a0 += part[(size_t(c) * pieces + p) * 2];
    a1 += part[(size_t(c) * pieces + p) * 2 + 1];
  }
  s0 = wave_reduce(a0);
  s1 = wave_reduce(a1);
  return lane == 0;
}

// batchnorm_mean_var finalize: the formulas of nn_batchnorm_mean_var.hlsl:46-59
// (one-pass var = max(0, E[x^2] - E[x]^2), unbiased running var
// var*m/max(1, m-1), momentum update), evaluated in double.
__device__ __forceinline__ void bn_stats_store(uint32_t c, double s0, double s1, uint32_t m,
                                               Buf mean, Buf var, Buf rmean, Buf rvar,
                                               uint32_t training, float momentum) {
  const double mu = s0 / m;
  const double v = fmax(0.0, s1 / m - mu * mu);
  st(mean, c, float(mu));
  st(var, c, float(v));
  if (training == 1) {
    const double unb = v * (double(m) / fmax(1.0, double(m) - 1.0));
    const double mo = momentum;
    st(rmean, c, float((1.0 - mo) * ld(rmean, c) + mo * mu));
    st(rvar, c, float((1.0 - mo) * ld(rvar, c) + mo * unb));
  }
}
__global__ void __launch_bounds__(256)
    k_bn_stats_final(const double* part, uint32_t pieces, uint32_t C, uint32_t m, Buf mean,
                     Buf var, Buf rmean, Buf rvar, uint32_t training, float momentum) {
  uint32_t c;
  double s0, s1;
  if (!bn_piece_sums(part, pieces, C, c, s0, s1)) return;
  bn_stats_store(c, s0, s1, m, mean, var, rmean, rvar, training, momentum);
}
// The same finish over the thousands of pieces a conv forward's GEMM leaves
// (one per column tile): a workgroup per channel, thread t adding pieces t,
// t + 256, ..., then the block tree, in a fixed order.
__global__ void __launch_bounds__(256)
    k_bn_stats_final_wide(const double* part, uint32_t pieces, uint32_t m, Buf mean, Buf var,
                          Buf rmean, Buf rvar, uint32_t training, float momentum) {
  __shared__ double sh[4];
  const uint32_t c = blockIdx.x;
  const double2* pc = reinterpret_cast<const double2*>(part) + size_t(c) * pieces;
  double a0 = 0.0, a1 = 0.0;
  // Eight loads in flight per thread (a conv's 4096 pieces per channel are
  // 16 per thread), added in piece order.
  for (uint32_t p0 = threadIdx.x; p0 < pieces; p0 += 256 * 8) {
    double2 e[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const uint32_t p = p0 + u * 256;
      e[u] = p < pieces ? pc[p] : double2{0.0, 0.0};
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      a0 += e[u].x;
      a1 += e[u].y;
    }
  }
  const double s0 = block_sum256(a0, sh);
  const double s1 = block_sum256(a1, sh);
  if (threadIdx.x == 0) bn_stats_store(c, s0, s1, m, mean, var, rmean, rvar, training, momentum);
}
__global__ void __launch_bounds__(256)
    k_bn_grad_final(const double* part, uint32_t pieces, uint32_t C, Buf dgamma, Buf dbeta) {
  uint32_t c;
  double s0, s1;
  if (!bn_piece_sums(part, pieces, C, c, s0, s1)) return;
  st(dgamma, c, float(s0));
  st(dbeta, c, float(s1));
}

static bool bn_reduce(const char* what, int mode, const Dispatch& d, Buf x, Buf dy, Buf mean,
                      Buf var, float eps, uint32_t N, uint32_t C, uint32_t S, double** partOut,
                      BnPieces* pcOut) {
  BnPieces pc = bn_pieces(N, C, S);
  const uint64_t total = uint64_t(N) * C * S;
  if (!total || total >= (1ull << 31)) {
    if (total) set_error("%s: tensor too large", what);
    return false;
  }
  double* part = reinterpret_cast<double*>(workspace(size_t(C) * pc.pieces * 4));
  if (!part) return false;
  const bool fast = covers(x, total) && (mode == 0 || covers(dy, total));
  dim3 grid(pc.pieces, C);
  FastDiv dS = make_fastdiv(S);
  if (fast && S % 4 == 0 && (reinterpret_cast<uintptr_t>(x.p) & 15) == 0 &&
      (mode == 0 || (reinterpret_cast<uintptr_t>(dy.p) & 15) == 0) &&
      (mode == 0 || (covers(mean, C) && covers(var, C)))) {
    const uint32_t S4 = S / 4, len4 = N * S4;
    const FastDiv dS4 = make_fastdiv(S4);
    const bool nt = stream_nt((mode == 0 ? 4.0 : 8.0) * double(total));
#define DCE_BNP(M, NT)                                                                         \
  hipLaunchKernelGGL((k_bn_partial4<M, NT, kBnUnroll>), dim3(C, pc.pieces), dim3(256), 0,       \
                     stream(), x.p,                                                            \
                     M ? dy.p : nullptr, M ? mean.p : nullptr, M ? var.p : nullptr, eps, C, S4, \
                     len4, pc.pieces, dS4, part)
    if (mode == 0 && nt) DCE_BNP(0, true);
    else if (mode == 0) DCE_BNP(0, false);
    else if (nt) DCE_BNP(1, true);
    else DCE_BNP(1, false);
#undef DCE_BNP
    *partOut = part;
    *pcOut = pc;
    return check_launch(what);
  }
  if (mode == 0) {
    if (fast)
      hipLaunchKernelGGL((k_bn_partial<0, false>), grid, dim3(256), 0, stream(), x, dy, mean, var,
                         eps, C, S, pc.len, pc.pieces, dS, part);
    else
      hipLaunchKernelGGL((k_bn_partial<0, true>), grid, dim3(256), 0, stream(), x, dy, mean, var,
                         eps, C, S, pc.len, pc.pieces, dS, part);
  } else {
    if (fast)
      hipLaunchKernelGGL((k_bn_partial<1, false>), grid, dim3(256), 0, stream(), x, dy, mean, var,
                         eps, C, S, pc.len, pc.pieces, dS, part);
    else
      hipLaunchKernelGGL((k_bn_partial<1, true>), grid, dim3(256), 0, stream(), x, dy, mean, var,
                         eps, C, S, pc.len, pc.pieces, dS, part);
  }
  (void)d;
  *partOut = part;
  *pcOut = pc;
  return check_launch(what);
}

// relu_grad / relu6_grad over the output z of a batch norm whose operands
// are unchanged since its forward: dz comes with the partial sums of that
// batch norm's backward reduce over (x, dz), so that the reduce only adds
// them up (bn_backward_reduce_fused).
template <int MODE>
static bool act_grad_bn(const char* what, const Dispatch& d) {
  if (d.nS < 2 || !d.nU) return false;
  BnLink L;
  if (!bn_link_of(d.srvs[1], &L)) return false;
  const uint64_t total = uint64_t(L.N) * L.C * L.S;
  const Buf g = S(d, 0), z = S(d, 1), out = U(d, 0);
  const auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (CU(d, 0) != total || L.S % 4 || !covers(g, total) || !covers(z, total) ||
      !covers(out, total) || !al16(g.p) || !al16(z.p) || !al16(out.p) || !al16(L.x) ||
      total >= (1ull << 31))
    return false;
  const BnPieces pc = bn_pieces(L.N, L.C, L.S);
  const uint64_t side_n = uint64_t(L.C) * pc.pieces * 4;
  Buffer* side = side_n < 0xFFFFFFFFull
                     ? static_cast<Buffer*>(create_buffer(nullptr, uint32_t(side_n)))
                     : nullptr;
  if (!side) return false;
  ProfScope prof(what, 0, 16.0 * double(total));
  const uint32_t S4 = L.S / 4, len4 = L.N * S4;
  double* part = reinterpret_cast<double*>(side->ptr);
  if (stream_nt(16.0 * double(total)))
    hipLaunchKernelGGL((k_bn_partial4<MODE, true, kBnUnroll>), dim3(L.C, pc.pieces), dim3(256), 0,
                       stream(), L.x, g.p, L.mean, L.var, L.eps, L.C, S4, len4, pc.pieces,
                       make_fastdiv(S4), part, z.p, out.p);
  else
    hipLaunchKernelGGL((k_bn_partial4<MODE, false, kBnUnroll>), dim3(L.C, pc.pieces), dim3(256),
                       0, stream(), L.x, g.p, L.mean, L.var, L.eps, L.C, S4, len4, pc.pieces,
                       make_fastdiv(S4), part, z.p, out.p);
  if (!check_launch(what)) {
    release_buffer(side);
    return false;
  }
  tag_bn_grad_part(d.uavs[0], d.srvs[1], side, pc.pieces);
  return true;
}
static bool sh_relu_grad(const Dispatch& d) {
  if (act_grad_bn<2>("relu_grad", d)) return true;
  return run_ew("relu_grad", OpReluGrad{}, U(d, 0), S(d, 0), S(d, 1), CU(d, 0), false);
}
static bool sh_relu6_grad(const Dispatch& d) {
  if (act_grad_bn<3>("relu6_grad", d)) return true;
  return run_ew("relu6_grad", OpRelu6Grad{}, U(d, 0), S(d, 0), S(d, 1), CU(d, 0), false);
}

static bool sh_bn_mean_var(const Dispatch& d) {
  uint32_t N = CU(d, 0), C = CU(d, 1), Sz = CU(d, 2), training = CU(d, 3);
  float momentum = CF(d, 4);
  if (!N || !C || !Sz) return true;
  // x straight from a conv forward that left its statistics: finish those.
  const Buffer* X = d.nS ? static_cast<const Buffer*>(d.srvs[0]) : nullptr;
  if (X && X->magic == kMagicLive && X->tag == kBnStatsTag && X->side && X->meta[0] == N &&
      X->meta[1] == C && X->meta[2] == Sz) {
    ProfScope prof("bn_stats_side", 0, 16.0 * double(C) * X->aux32);
    hipLaunchKernelGGL(k_bn_stats_final_wide, dim3(C), dim3(256), 0, stream(),
                       reinterpret_cast<const double*>(X->side->ptr), X->aux32, N * Sz, U(d, 0),
                       U(d, 1), U(d, 2), U(d, 3), training, momentum);
    if (!check_launch("batchnorm_mean_var")) return false;
  } else {
    double* part;
    BnPieces pc;
    ProfScope prof("bn_stats", 0, 4.0 * double(N) * C * Sz);
    if (!bn_reduce("batchnorm_mean_var", 0, d, S(d, 0), Buf{nullptr, 0}, Buf{nullptr, 0},
                   Buf{nullptr, 0}, 0.f, N, C, Sz, &part, &pc))
      return false;
    hipLaunchKernelGGL(k_bn_stats_final, dim3(cdiv(C, 4)), dim3(256), 0, stream(), part,
                       pc.pieces, C, N * Sz, U(d, 0), U(d, 1), U(d, 2), U(d, 3), training,
                       momentum);
    if (!check_launch("batchnorm_mean_var")) return false;
  }
  // The statistics, tagged so that the backward can tell they are unchanged.
  if (d.nU >= 2) tag_bn_moments(d.uavs[0], d.uavs[1]);
  return true;
}

static bool sh_bn_backward_reduce(const Dispatch& d) {
  uint32_t N = CU(d, 0), C = CU(d, 1), Sz = CU(d, 2);
  float eps = CF(d, 3);
  if (!N || !C || !Sz) return true;
  // dy made by relu_grad / relu6_grad over this batch norm's output, with
  // the partial sums for exactly these operands: add them up.
  if (d.nS >= 4 && d.nU >= 2) {
    uint32_t pieces = 0;
    if (const double* gp = bn_grad_part_of(d.srvs[1], d.srvs[0], d.srvs[2], d.srvs[3], N, C, Sz,
                                           eps, &pieces)) {
      ProfScope prof("bn_bwd_reduce_side", 0, 16.0 * double(C) * pieces);
      hipLaunchKernelGGL(k_bn_grad_final, dim3(cdiv(C, 4)), dim3(256), 0, stream(), gp, pieces, C,
                         U(d, 0), U(d, 1));
      return check_launch("batchnorm_backward_reduce");
    }
  }
  double* part;
  BnPieces pc;
  ProfScope prof("bn_bwd_reduce", 0, 8.0 * double(N) * C * Sz);
  if (!bn_reduce("batchnorm_backward_reduce", 1, d, S(d, 0), S(d, 1), S(d, 2), S(d, 3), eps, N, C,
                 Sz, &part, &pc))
    return false;
  hipLaunchKernelGGL(k_bn_grad_final, dim3(cdiv(C, 4)), dim3(256), 0, stream(), part,
                     pc.pieces, C, U(d, 0), U(d, 1));
  return check_launch("batchnorm_backward_reduce");
}

// y = (x - mu) * rstd * gamma + beta   (nn_batchnorm_forward.hlsl:24-34)
// dx = (gamma*rstd) * (dy - (dbeta + xhat*dgamma)/m)   (nn_batchnorm_backward_dx.hlsl:26-38)
template <int MODE, bool CHECK>
__global__ void k_bn_elem(Buf x, Buf dy, Buf mean, Buf var, Buf gamma, Buf beta_or_dg, Buf dbeta,
                          Buf out, float eps, uint32_t C, uint32_t total, FastDiv dS,
                          FastDiv dC, float m) {
  const uint32_t i = gtid();
  if (i >= total) return;
  const uint32_t q = fdiv(i, dS);
  const uint32_t c = q - fdiv(q, dC) * C;
  const float mu = ld(mean, c);
  const float rstd = 1.0f / sqrtf(ld(var, c) + eps);
  const float xv = CHECK ? ld(x, i) : x.p[i];
  const float xh = (xv - mu) * rstd;
  if (MODE == 0) {
    const float v = xh * ld(gamma, c) + ld(beta_or_dg, c);
    if (CHECK) st(out, i, v); else out.p[i] = v;
  } else {
    const float g = ld(gamma, c), dg = ld(beta_or_dg, c), db = ld(dbeta, c);
    const float dyv = CHECK ? ld(dy, i) : dy.p[i];
    const float v = bn_dx_elem(xv, dyv, mu, rstd, g, dg, db, m);
    if (CHECK) st(out, i, v); else out.p[i] = v;
  }
}
// Quad form (S % 4 == 0, every buffer covering its size): the four elements
// of a quad share a channel, whose parameters are computed once.  ACT (the
// forward only): also store ACT(y) to act_out (1: relu, 2: relu6, with the
// relu / relu6 shaders' own functors), for the activation that follows.
template <int MODE, bool NT, int ACT = 0>
__global__ void __launch_bounds__(256)
    k_bn_elem4(const float* __restrict__ x, const float* __restrict__ dy,
               const float* __restrict__ mean, const float* __restrict__ var,
               const float* __restrict__ gamma, const float* __restrict__ beta_or_dg,
               const float* __restrict__ dbeta, float* __restrict__ out, float eps, uint32_t C,
               uint32_t total4, FastDiv dS4, FastDiv dC, float m,
               float* __restrict__ act_out = nullptr) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= total4) return;
  const uint32_t q = fdiv(i, dS4);
  const uint32_t c = q - fdiv(q, dC) * C;
  const float mu = mean[c];
  const float rstd = 1.0f / sqrtf(var[c] + eps);
  const f4 xv = ld4s<NT>(x + size_t(i) * 4);
  f4 r;
  if (MODE == 0) {
    const float g = gamma[c], b = beta_or_dg[c];
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = (xv[e] - mu) * rstd * g + b;
  } else {
    const float g = gamma[c], dg = beta_or_dg[c], db = dbeta[c];
    const f4 gv = ld4s<NT>(dy + size_t(i) * 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = bn_dx_elem(xv[e], gv[e], mu, rstd, g, dg, db, m);
  }
  st4s<NT>(out + size_t(i) * 4, r);
  if constexpr (ACT != 0) {
    f4 a;
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = ACT == 1 ? OpRelu{}(r[e], 0.f) : OpRelu6{}(r[e], 0.f);
    st4s<NT>(act_out + size_t(i) * 4, a);
  }
}

template <int MODE>
static bool bn_elem(const char* what, const Dispatch& d) {
  uint32_t N = CU(d, 0), C = CU(d, 1), Sz = CU(d, 2);
  float eps = CF(d, 3);
  uint64_t total = uint64_t(N) * C * Sz;
  if (!total) return true;
  if (total >= (1ull << 31)) {
    set_error("%s: tensor too large", what);
    return false;
  }
  Buf x = S(d, 0);
  Buf dy = MODE == 1 ? S(d, 1) : Buf{nullptr, 0};
  Buf mean = MODE == 1 ? S(d, 2) : S(d, 1);
  Buf var = MODE == 1 ? S(d, 3) : S(d, 2);
  Buf gamma = MODE == 1 ? S(d, 4) : S(d, 3);
  Buf b2 = MODE == 1 ? S(d, 5) : S(d, 4);
  Buf db = MODE == 1 ? S(d, 6) : Buf{nullptr, 0};
  Buf out = U(d, 0);
  const bool fast = covers(x, total) && covers(out, total) && (MODE == 0 || covers(dy, total));
  const auto al16 = [](const Buf& b) { return (reinterpret_cast<uintptr_t>(b.p) & 15) == 0; };
  const bool quad = fast && Sz % 4 == 0 && al16(x) && al16(out) && (MODE == 0 || al16(dy)) &&
                    covers(mean, C) && covers(var, C) && covers(gamma, C) && covers(b2, C) &&
                    (MODE == 0 || covers(db, C));
  // The activation that followed this batch norm (same gamma) last time is
  // stored as well (quad form of the forward), into a buffer that the
  // activation's call adopts as its output (bn_act_adopt) instead of running.
  const uint32_t act = MODE == 0 && quad && d.nS >= 4 && d.nU ? bn_act_guess(d.srvs[3]) : 0;
  ProfScope prof(MODE == 0 ? "bn_fwd" : "bn_bwd_dx", 0,
                 (MODE == 0 && !act ? 8.0 : 12.0) * double(total));
  if (quad) {
    const uint32_t total4 = uint32_t(total / 4);
    if constexpr (MODE == 0) {
      Buffer* side = act ? static_cast<Buffer*>(create_buffer(nullptr, uint32_t(total))) : nullptr;
      if (side) {
        const bool nt = stream_nt(12.0 * double(total));
#define DCE_BNA(A, NTV)                                                                         \
  hipLaunchKernelGGL((k_bn_elem4<0, NTV, A>), dim3(cdiv(total4, 256)), dim3(256), 0, stream(),  \
                     x.p, dy.p, mean.p, var.p, gamma.p, b2.p, db.p, out.p, eps, C, total4,      \
                     make_fastdiv(Sz / 4), make_fastdiv(C), float(uint64_t(N) * Sz), side->ptr)
        if (act == 1 && nt) DCE_BNA(1, true);
        else if (act == 1) DCE_BNA(1, false);
        else if (nt) DCE_BNA(2, true);
        else DCE_BNA(2, false);
#undef DCE_BNA
        if (!check_launch(what)) {
          release_buffer(side);
          return false;
        }
        tag_bn_out(d.uavs[0], d.srvs[0], d.srvs[1], d.srvs[3], side, act, N, C, Sz, eps);
        return true;
      }
      if (d.nS >= 4 && d.nU)
        tag_bn_out(d.uavs[0], d.srvs[0], d.srvs[1], d.srvs[3], nullptr, 0, N, C, Sz, eps);
    }
    if (stream_nt((MODE == 1 ? 12.0 : 8.0) * double(total)))
      hipLaunchKernelGGL((k_bn_elem4<MODE, true>), dim3(cdiv(total4, 256)), dim3(256), 0,
                         stream(), x.p, dy.p, mean.p, var.p, gamma.p, b2.p, db.p, out.p, eps, C,
                         total4, make_fastdiv(Sz / 4), make_fastdiv(C), float(uint64_t(N) * Sz));
    else
      hipLaunchKernelGGL((k_bn_elem4<MODE, false>), dim3(cdiv(total4, 256)), dim3(256), 0,
                         stream(), x.p, dy.p, mean.p, var.p, gamma.p, b2.p, db.p, out.p, eps, C,
                         total4, make_fastdiv(Sz / 4), make_fastdiv(C), float(uint64_t(N) * Sz));
    return check_launch(what);
  }
  dim3 grid(cdiv(total, 256));
  if (fast)
    hipLaunchKernelGGL((k_bn_elem<MODE, false>), grid, dim3(256), 0, stream(), x, dy, mean, var,
                       gamma, b2, db, out, eps, C, uint32_t(total), make_fastdiv(Sz),
                       make_fastdiv(C), float(uint64_t(N) * Sz));
  else
    hipLaunchKernelGGL((k_bn_elem<MODE, true>), grid, dim3(256), 0, stream(), x, dy, mean, var,
                       gamma, b2, db, out, eps, C, uint32_t(total), make_fastdiv(Sz),
                       make_fastdiv(C), float(uint64_t(N) * Sz));
  return check_launch(what);
}
static bool sh_bn_forward(const Dispatch& d) { return bn_elem<0>("batchnorm_forward", d); }
// Over the output of a conv whose backward reads an NHWC G (the forward's
// tag says so), dx comes with that G and its bias-gradient partials (owned
// by dx, kGradGTag), and the conv backward then runs no transpose pass.
static bool sh_bn_backward_dx(const Dispatch& d) {
  const uint32_t N = CU(d, 0), C = CU(d, 1), Sz = CU(d, 2);
  const float eps = CF(d, 3);
  const Buffer* X = d.nS >= 7 ? static_cast<const Buffer*>(d.srvs[0]) : nullptr;
  if (N && C && Sz && d.nU && X && X->magic == kMagicLive && X->tag == kBnStatsTag &&
      X->meta[0] == N && X->meta[1] == C && X->meta[2] == Sz && X->meta[3] &&
      uint64_t(X->meta[3]) * X->meta[4] == Sz) {
    const uint64_t total = uint64_t(N) * C * Sz;
    const Buf x = S(d, 0), dy = S(d, 1), mean = S(d, 2), var = S(d, 3), gamma = S(d, 4),
              dg = S(d, 5), db = S(d, 6), out = U(d, 0);
    const size_t nG = g_side_floats(kGLayoutNhwc, N, C, X->meta[3], X->meta[4]);
    const uint32_t rows = bn_dx_g_rows(N, C, Sz);
    const uint64_t side_n = nG + uint64_t(rows) * C;
    if (covers(x, total) && covers(dy, total) && covers(out, total) && covers(mean, C) &&
        covers(var, C) && covers(gamma, C) && covers(dg, C) && covers(db, C) &&
        side_n < 0xFFFFFFFFull) {
      Buffer* side = static_cast<Buffer*>(create_buffer(nullptr, uint32_t(side_n)));
      if (side) {
        if (!bn_dx_g(x.p, dy.p, mean.p, var.p, gamma.p, dg.p, db.p, eps, out.p, side->ptr,
                     side->ptr + nG, N, C, Sz)) {
          release_buffer(side);
          return false;
        }
        tag_grad_g_nhwc(d.uavs[0], side, N, C, X->meta[3], X->meta[4], rows);
        return true;
      }
    }
  }
  return bn_elem<1>("batchnorm_backward_dx", d);
}

// ===========================================================================
// Max pooling
// ===========================================================================
__global__ void k_maxpool_fwd(Buf x, Buf out, Buf idx, uint32_t BC, uint32_t H, uint32_t W,
                              uint32_t k, uint32_t s, uint32_t OH, uint32_t OW) {
  const uint32_t o = gtid();
  if (o >= BC * OH * OW) return;
  const uint32_t ow = o % OW, t = o / OW, oh = t % OH, bc = t / OH;
  const uint32_t base = bc * H * W;
  float mx = -1e30f;
  uint32_t mi = 0xFFFFFFFFu;
  for (uint32_t ph = 0; ph < k; ++ph) {
    const uint32_t ih = oh * s + ph;
    for (uint32_t pw = 0; pw < k; ++pw) {
      const uint32_t iw = ow * s + pw;
      if (ih < H && iw < W) {
        const uint32_t ii = base + ih * W + iw;
        const float v = ld(x, ii);
        if (v > mx) {
          mx = v;
          mi = ii;
        }
      }
    }
  }
  st(out, o, mx);
  st(idx, o, __uint_as_float(mi));
}

// Fused-path forward for windows that lie inside the input (floor mode):
// K x K window unrolled, every load unconditional, same first-max rule.
template <int K>
__global__ void k_maxpool_fwd_k(const float* __restrict__ x, float* __restrict__ out,
                                uint32_t* __restrict__ idx, uint32_t total, uint32_t H, uint32_t W,
                                uint32_t s, uint32_t OH, uint32_t OW, FastDiv dOW, FastDiv dOH,
                                uint32_t nx) {
  const uint32_t o = gtid();
  if (o >= total) return;
  const uint32_t t = fdiv(o, dOW);
  const uint32_t ow = o - t * OW;
  const uint32_t bc = fdiv(t, dOH);
  const uint32_t oh = t - bc * OH;
  const uint32_t base = bc * H * W + oh * s * W + ow * s;
  // Each window row is one 8-byte (K = 2) or 16-byte (K = 3) load.  Rows of
  // odd length leave these only 4-byte aligned; the GPU runs with unaligned
  // access enabled.  The 16-byte load also reads the column after the
  // window, so the last window of the buffer reads dword by dword.
  float v[K][K];
  if (K == 2 || base + (K - 1) * W + 3 < nx) {
#pragma unroll
    for (int a = 0; a < K; ++a) {
      const float* r = x + base + a * W;
      if constexpr (K == 2) {
        const f2 q = ldu<f2>(r);
        v[a][0] = q[0];
        v[a][1] = q[1];
      } else {
        const f4 q = ldu<f4>(r);
#pragma unroll
        for (int b = 0; b < K; ++b) v[a][b] = q[b];
      }
    }
  } else {
#pragma unroll
    for (int a = 0; a < K; ++a)
#pragma unroll
      for (int b = 0; b < K; ++b) v[a][b] = x[base + a * W + b];
  }
  float mx = -1e30f;
  uint32_t mi = 0xFFFFFFFFu;
#pragma unroll
  for (int a = 0; a < K; ++a)
#pragma unroll
    for (int b = 0; b < K; ++b)
      if (v[a][b] > mx) {
        mx = v[a][b];
        mi = base + a * W + b;
      }
  out[o] = mx;
  idx[o] = mi;
}

bool maxpool_forward(const float* x, float* out, float* idx, uint32_t B, uint32_t C, uint32_t H,
                     uint32_t W, uint32_t k, uint32_t s, uint32_t OH, uint32_t OW) {
  const uint32_t n = B * C * OH * OW;
  ProfScope prof("maxpool_fwd", 0, 4.0 * double(B) * C * H * W + 8.0 * n);
  const bool inside = n && s && (OH - 1) * s + k <= H && (OW - 1) * s + k <= W;
  if (inside && (k == 2 || k == 3)) {
    uint32_t* ip = reinterpret_cast<uint32_t*>(idx);
    const FastDiv fOW = make_fastdiv(OW), fOH = make_fastdiv(OH);
    const uint32_t nx = B * C * H * W;
    if (k == 2)
      hipLaunchKernelGGL(k_maxpool_fwd_k<2>, dim3(cdiv(n, 256)), dim3(256), 0, stream(), x, out, ip,
                         n, H, W, s, OH, OW, fOW, fOH, nx);
    else
      hipLaunchKernelGGL(k_maxpool_fwd_k<3>, dim3(cdiv(n, 256)), dim3(256), 0, stream(), x, out, ip,
                         n, H, W, s, OH, OW, fOW, fOH, nx);
    return check_launch("maxpool_forward");
  }
  hipLaunchKernelGGL(k_maxpool_fwd, dim3(cdiv(n, 256)), dim3(256), 0, stream(),
                     Buf{const_cast<float*>(x), B * C * H * W}, Buf{out, n}, Buf{idx, n}, B * C,
                     H, W, k, s, OH, OW);
  return check_launch("maxpool_forward");
}

// Deterministic gather: every input element sums dZ over the windows that
// contain it and whose recorded argmax is this element, in (oh, ow) order.
__global__ void k_maxpool_bwd_gather(const float* __restrict__ dz, const uint32_t* __restrict__ idx,
                                     float* __restrict__ dx, uint32_t total, uint32_t H, uint32_t W,
                                     uint32_t k, uint32_t s, uint32_t OH, uint32_t OW,
                                     FastDiv dW, FastDiv dH) {
  const uint32_t i = gtid();
  if (i >= total) return;
  const uint32_t t = fdiv(i, dW);
  const uint32_t iw = i - t * W;
  const uint32_t bc = fdiv(t, dH);
  const uint32_t ih = t - bc * H;
  const uint32_t ohlo = (ih + 1 >= k) ? (ih + 1 - k + s - 1) / s : 0;
  const uint32_t ohhi = min(ih / s, OH - 1);
  const uint32_t owlo = (iw + 1 >= k) ? (iw + 1 - k + s - 1) / s : 0;
  const uint32_t owhi = min(iw / s, OW - 1);
  float acc = 0.f;
  const uint32_t ob = bc * OH * OW;
  for (uint32_t oh = ohlo; oh <= ohhi; ++oh)
    for (uint32_t ow = owlo; ow <= owhi; ++ow) {
      const uint32_t o = ob + oh * OW + ow;
      if (idx[o] == i) acc += dz[o];
    }
  dx[i] = acc;
}
// Same gather with at most NW windows per axis covering an input element
// (NW = ceil(k / s)): all NW*NW (index, value) pairs are loaded up front from
// clamped in-plane addresses, then the matching ones are added in (oh, ow)
// order -- no load waits on a compare.
template <int NW>
__global__ void k_maxpool_bwd_gather_n(const float* __restrict__ dz,
                                       const uint32_t* __restrict__ idx, float* __restrict__ dx,
                                       uint32_t total, uint32_t H, uint32_t W, uint32_t k,
                                       uint32_t OH, uint32_t OW, FastDiv dW, FastDiv dH,
                                       FastDiv dS) {
  const uint32_t i = gtid();
  if (i >= total) return;
  const uint32_t t = fdiv(i, dW);
  const uint32_t iw = i - t * W;
  const uint32_t bc = fdiv(t, dH);
  const uint32_t ih = t - bc * H;
  const uint32_t s = dS.d;
  const uint32_t ohlo = (ih + 1 >= k) ? fdiv(ih + 1 - k + s - 1, dS) : 0;
  const uint32_t ohhi = min(fdiv(ih, dS), OH - 1);
  const uint32_t owlo = (iw + 1 >= k) ? fdiv(iw + 1 - k + s - 1, dS) : 0;
  const uint32_t owhi = min(fdiv(iw, dS), OW - 1);
  const uint32_t ob = bc * OH * OW;
  uint32_t id[NW][NW];
  float v[NW][NW];
#pragma unroll
  for (int a = 0; a < NW; ++a)
#pragma unroll
    for (int b = 0; b < NW; ++b) {
      const uint32_t o = ob + min(ohlo + a, OH - 1) * OW + min(owlo + b, OW - 1);
      id[a][b] = idx[o];
      v[a][b] = dz[o];
    }
  float acc = 0.f;
#pragma unroll
  for (int a = 0; a < NW; ++a)
#pragma unroll
    for (int b = 0; b < NW; ++b)
      if (ohlo + a <= ohhi && owlo + b <= owhi && id[a][b] == i) acc += v[a][b];
  dx[i] = acc;
}

// The windows covering the S x S input block (a, b) of one plane: a thread
// owns the block and loads the NW x NW windows o in [a - (K-1)/S, a] x
// [b - (K-1)/S, b] once, as (argmax index, value) pairs; with MASK also each
// window's maximum.  A window whose recorded argmax is input i necessarily
// contains i, so every input of the block adds the values of the matching
// windows, in (oh, ow) order (sum).
// PAIR (NW == 2, OW >= 2): the two window columns b-1, b of a window row are
// one 8-byte load at column ps = clamp(b-1, 0, OW-2).  These addresses are
// only 4-byte aligned when rows have odd length; the GPU runs with unaligned
// access enabled, and halving the memory instructions takes the AlexNet
// 55x55 backward from 35 to 25 us (warm) and 51 to 38 us (cold caches).
// MASK (a max-pool over a ReLU conv output): the maximum of a window is the
// conv output at its argmax, so the conv backward's mask (output <= 0 ->
// gradient 0) is known per window: sum<true> adds only the windows whose
// maximum is not <= 0.  Every window routed to input i has the same maximum
// (that input's value), so sum<true>(i) is either sum<false>(i), bit for bit,
// or 0.
template <int K, int S, bool PAIR, bool MASK>
struct PoolWin {
  static constexpr int NW = (K - 1) / S + 1;
  static_assert(!PAIR || (NW == 2 && S == 2), "pair loads cover two window columns");
  uint32_t id[NW][NW];
  float v[NW][NW];
  bool keep[NW][NW];

  __device__ __forceinline__ void load(const float* __restrict__ dz,
                                       const uint32_t* __restrict__ idx,
                                       const float* __restrict__ pooled, uint32_t plane,
                                       uint32_t a, uint32_t b, uint32_t OH, uint32_t OW) {
    if constexpr (PAIR) {
      typedef uint32_t u2 __attribute__((ext_vector_type(2)));
      const uint32_t ps = min(max(int(b) - 1, 0), int(OW) - 2);
      const bool lok = b >= 1, rok = b < OW;
      const bool li = b == OW, ri = b != 0;  // element of the pair holding column b-1 / b
#pragma unroll
      for (int wa = 0; wa < NW; ++wa) {
        const int oh = int(a) - (NW - 1) + wa;
        const bool hok = oh >= 0 && oh < int(OH);
        const uint32_t o = (plane * OH + uint32_t(hok ? oh : 0)) * OW + ps;
        const u2 iv = ldu<u2>(idx + o);
        const f2 dv = ldu<f2>(dz + o);
        id[wa][0] = (hok && lok) ? (li ? iv[1] : iv[0]) : 0xFFFFFFFFu;
        id[wa][1] = (hok && rok) ? (ri ? iv[1] : iv[0]) : 0xFFFFFFFFu;
        v[wa][0] = li ? dv[1] : dv[0];
        v[wa][1] = ri ? dv[1] : dv[0];
        if constexpr (MASK) {
          const f2 pv = ldu<f2>(pooled + o);
          keep[wa][0] = !((li ? pv[1] : pv[0]) <= 0.f);
          keep[wa][1] = !((ri ? pv[1] : pv[0]) <= 0.f);
        }
      }
    } else {
#pragma unroll
      for (int wa = 0; wa < NW; ++wa) {
        const int oh = int(a) - (NW - 1) + wa;
#pragma unroll
        for (int wb = 0; wb < NW; ++wb) {
          const int ow = int(b) - (NW - 1) + wb;
          const bool ok = oh >= 0 && oh < int(OH) && ow >= 0 && ow < int(OW);
          const uint32_t o = (plane * OH + uint32_t(ok ? oh : 0)) * OW + uint32_t(ok ? ow : 0);
          const uint32_t iv = idx[o];
          v[wa][wb] = dz[o];
          id[wa][wb] = ok ? iv : 0xFFFFFFFFu;
          if constexpr (MASK) keep[wa][wb] = !(pooled[o] <= 0.f);
        }
      }
    }
  }

  template <bool KEEP>
  __device__ __forceinline__ float sum(uint32_t i) const {
    float acc = 0.f;
#pragma unroll
    for (int wa = 0; wa < NW; ++wa)
#pragma unroll
      for (int wb = 0; wb < NW; ++wb)
        if (id[wa][wb] == i && (!KEEP || keep[wa][wb])) acc += v[wa][wb];
    return acc;
  }
};

// Stores input row ih's S = 2 gradients of block column b: one 8-byte store
// when the pair lies in the row (aligned for rows of even length; PAIR also
// takes odd ones).
template <bool PAIR>
__device__ __forceinline__ void store_pair_row(float* __restrict__ row, uint32_t b, uint32_t W,
                                               float o0, float o1) {
  if (2 * b + 1 < W && (PAIR || (W & 1) == 0)) {
    stu(row, f2{o0, o1});
  } else {
    row[0] = o0;
    if (2 * b + 1 < W) row[1] = o1;
  }
}

// Block form: a thread owns an S x S block of inputs (PoolWin) and writes
// its gradients, an output pair of a row as one 8-byte store whenever both
// lie in the row.
template <int K, int S, bool PAIR>
__global__ void k_maxpool_bwd_blk(const float* __restrict__ dz, const uint32_t* __restrict__ idx,
                                  float* __restrict__ dx, uint32_t items, uint32_t H, uint32_t W,
                                  uint32_t OH, uint32_t OW, uint32_t BH, uint32_t BW,
                                  FastDiv dBW, FastDiv dBH) {
  const uint32_t item = blockIdx.x * 256 + threadIdx.x;
  if (item >= items) return;
  const uint32_t t = fdiv(item, dBW), b = item - t * BW;
  const uint32_t plane = fdiv(t, dBH), a = t - plane * BH;
  PoolWin<K, S, PAIR, false> pw;
  pw.load(dz, idx, nullptr, plane, a, b, OH, OW);
#pragma unroll
  for (int r = 0; r < S; ++r) {
    const uint32_t ih = a * S + r;
    if (ih >= H) continue;
    const uint32_t i0 = (plane * H + ih) * W + b * S;
    float o[S];
#pragma unroll
    for (int c = 0; c < S; ++c) o[c] = pw.template sum<false>(i0 + c);
    float* row = dx + i0;
    if constexpr (S == 2) {
      store_pair_row<PAIR>(row, b, W, o[0], o[1]);
    } else {
#pragma unroll
      for (int c = 0; c < S; ++c)
        if (b * S + c < W) row[c] = o[c];
    }
  }
}

// Max-pool backward over a ReLU conv output whose backward reads its masked
// gradient on the padded pixel grid (kGLayoutPad, the stride-phase dW): dx
// as k_maxpool_bwd_blk (S = 2), and G_pad[plane][ih][iw] for iw < gw
// (= pad4(W); zero for iw >= W) with the bias-gradient partials.  One wave
// per (plane, chunk of 64 blocks): a wave's blocks lie in one plane, so the
// wave's G sum is one partial, db[c][b*nch + chunk].
template <int K, bool PAIR>
__global__ void __launch_bounds__(256)
    k_maxpool_bwd_gpad(const float* __restrict__ dz, const uint32_t* __restrict__ idx,
                       const float* __restrict__ pooled, float* __restrict__ dx,
                       float* __restrict__ gp, float* __restrict__ db, uint32_t C, uint32_t H,
                       uint32_t W, uint32_t OH, uint32_t OW, uint32_t gw, uint32_t BW,
                       uint32_t nblk, uint32_t nch, uint32_t nB, uint32_t waves, FastDiv dBW,
                       FastDiv dNch) {
  const uint32_t wv = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wv >= waves) return;  // whole waves
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t plane = fdiv(wv, dNch), chunk = wv - plane * nch;
  const uint32_t item = chunk * 64 + lane;
  const bool live = item < nblk;
  const uint32_t it = live ? item : 0u;
  const uint32_t a = fdiv(it, dBW), b = it - a * BW;
  PoolWin<K, 2, PAIR, true> pw;
  pw.load(dz, idx, pooled, plane, a, b, OH, OW);
  float sum = 0.f;
  if (live) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t ih = 2 * a + r;
      if (ih >= H) continue;
      const uint32_t i0 = (plane * H + ih) * W + 2 * b;
      const float o0 = pw.template sum<false>(i0), o1 = pw.template sum<false>(i0 + 1);
      const float m0 = pw.template sum<true>(i0);
      const float m1 = 2 * b + 1 < W ? pw.template sum<true>(i0 + 1) : 0.f;
      store_pair_row<PAIR>(dx + i0, b, W, o0, o1);
      float* grow = gp + (size_t(plane) * H + ih) * gw + 2 * b;  // 8-byte aligned: gw % 4 == 0
      *reinterpret_cast<f2*>(grow) = f2{m0, m1};
      if (b == BW - 1 && gw > 2 * BW) *reinterpret_cast<f2*>(grow + 2) = f2{0.f, 0.f};
      sum += m0 + m1;
    }
  }
  sum = wave_reduce(sum);
  if (lane == 0) {
    const uint32_t bi = plane / C, c = plane - bi * C;
    db[size_t(c) * nB * nch + size_t(bi) * nch + chunk] = sum;
  }
}

// 2 x 2 windows with stride 2 on planes of twice the output size (W a
// multiple of 4): a thread takes two neighbouring windows (ow = 2q, 2q + 1)
// with one 8-byte load of their indices and one of their values, and writes
// the 2 x 4 inputs they cover as two 16-byte stores.  Each input lies in
// exactly one window; it receives 0 + that window's value when the window's
// argmax is this input, else 0 (the sum of the block kernel, same bits).
__global__ void __launch_bounds__(256)
    k_maxpool_bwd_22q(const float* __restrict__ dz, const uint32_t* __restrict__ idx,
                      float* __restrict__ dx, uint32_t items, uint32_t OW2, FastDiv dOW2) {
  typedef uint32_t u2 __attribute__((ext_vector_type(2)));
  const uint32_t item = blockIdx.x * 256 + threadIdx.x;
  if (item >= items) return;
  const uint32_t t = fdiv(item, dOW2), q = item - t * OW2;  // t = plane * OH + oh
  const uint32_t o = t * (2 * OW2) + 2 * q;
  const u2 iv = *reinterpret_cast<const u2*>(idx + o);
  const f2 dv = *reinterpret_cast<const f2*>(dz + o);
  const uint32_t W = 4 * OW2;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    // Input row 2*oh + r of the plane: (plane * H + 2 * oh + r) * W = (2t + r) * W.
    const uint32_t i0 = (2 * t + r) * W + 4 * q;
    f4 out;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float acc = 0.f;
      if ((c < 2 ? iv[0] : iv[1]) == i0 + c) acc += c < 2 ? dv[0] : dv[1];
      out[c] = acc;
    }
    *reinterpret_cast<f4*>(dx + i0) = out;
  }
}

// Fallback when the pooling geometry is unknown (indices this library did
// not produce), for planes too large for k_maxpool_bwd_plane_lds below: one
// thread per (b, c) plane adds the plane's dZ values to
// dX[idx] in output order, after dX was cleared.  Every input then sums its
// windows in (oh, ow) order, as the gather kernels do, with no atomics.  An
// index outside its own plane cannot come from a pooling window; it is
// dropped, as is the no-argmax marker 0xFFFFFFFF.
__global__ void k_maxpool_bwd_planes(const float* __restrict__ dz, const uint32_t* __restrict__ idx,
                                     float* __restrict__ dx, uint32_t planes, uint32_t outPer,
                                     uint32_t inPer) {
  const uint32_t p = gtid();
  if (p >= planes) return;
  const uint32_t lo = p * inPer, hi = lo + inPer;
  for (uint32_t j = 0; j < outPer; ++j) {
    const uint32_t o = p * outPer + j;
    const uint32_t t = idx[o];
    if (t >= lo && t < hi) dx[t] += dz[o];
  }
}

// The same per-plane sum with one workgroup per plane and the plane's
// inputs accumulated in LDS (planes of at most kPlaneLds inputs).  The plane's
// outputs are taken 256 at a time, in output order; in each round the first
// lane of a target sums the round's contributions to that target in lane
// order onto the running value, so every input still adds its windows one by
// one in output order (((0 + a) + b) + c: the per-thread kernel's rounding),
// and each input is written once, with no clearing pass.  kPlaneLds keeps the
// dynamic LDS plus the two 1 KiB round arrays under 64 KiB.
constexpr uint32_t kPlaneLds = 14336;
__global__ void __launch_bounds__(256) k_maxpool_bwd_plane_lds(const float* __restrict__ dz,
                                                               const uint32_t* __restrict__ idx,
                                                               float* __restrict__ dx,
                                                               uint32_t outPer, uint32_t inPer) {
  extern __shared__ float acc[];
  __shared__ uint32_t tg[256];
  __shared__ float dv[256];
  const uint32_t tid = threadIdx.x;
  const uint64_t lo = uint64_t(blockIdx.x) * inPer;
  const uint64_t o0 = uint64_t(blockIdx.x) * outPer;
  for (uint32_t i = tid; i < inPer; i += 256) acc[i] = 0.f;
  for (uint32_t base = 0; base < outPer; base += 256) {
    const uint32_t j = base + tid;
    uint32_t t = 0xFFFFFFFFu;
    float v = 0.f;
    if (j < outPer) {
      const uint32_t g = idx[o0 + j];
      if (g >= lo && uint64_t(g) < lo + inPer) {
        t = uint32_t(g - lo);
        v = dz[o0 + j];
      }
    }
    tg[tid] = t;
    dv[tid] = v;
    __syncthreads();   // also orders the clear (first round) and the previous round's adds
    if (t != 0xFFFFFFFFu) {
      bool first = true;
      for (uint32_t l = 0; l < tid; ++l)
        if (tg[l] == t) {
          first = false;
          break;
        }
      if (first) {
        float a = acc[t];
        for (uint32_t l = tid; l < 256; ++l)
          if (tg[l] == t) a += dv[l];
        acc[t] = a;
      }
    }
    __syncthreads();
  }
  for (uint32_t i = tid; i < inPer; i += 256) dx[lo + i] = acc[i];
}

bool maxpool_backward(const float* dz, const float* idx, float* dx, uint32_t B, uint32_t C,
                      uint32_t OH, uint32_t OW, uint32_t xcount, uint32_t H, uint32_t W,
                      uint32_t k, uint32_t s) {
  const uint32_t n = B * C * OH * OW;
  ProfScope prof("maxpool_bwd", 0, 8.0 * n + 4.0 * xcount);
  const uint32_t* ip = reinterpret_cast<const uint32_t*>(idx);
  if (k && s && H && W) {
    if (n == 0) return fill_zero(dx, xcount);
    if (s == 2 && (k == 2 || k == 3) && xcount == B * C * H * W) {
      const uint32_t BH = cdiv(H, 2), BW = cdiv(W, 2), items = B * C * BH * BW;
      const dim3 grid(cdiv(items, 256));
      const FastDiv fBW = make_fastdiv(BW), fBH = make_fastdiv(BH);
      const bool quad = k == 2 && H == 2 * OH && W == 2 * OW && OW % 2 == 0 &&
                        (reinterpret_cast<uintptr_t>(dx) & 15) == 0 &&
                        (reinterpret_cast<uintptr_t>(dz) & 7) == 0 &&
                        (reinterpret_cast<uintptr_t>(ip) & 7) == 0;
      if (quad) {
        const uint32_t OW2 = OW / 2, n2 = B * C * OH * OW2;
        hipLaunchKernelGGL(k_maxpool_bwd_22q, dim3(cdiv(n2, 256)), dim3(256), 0, stream(), dz, ip,
                           dx, n2, OW2, make_fastdiv(OW2));
      } else if (k == 2)
        hipLaunchKernelGGL((k_maxpool_bwd_blk<2, 2, false>), grid, dim3(256), 0, stream(), dz,
                           ip, dx, items, H, W, OH, OW, BH, BW, fBW, fBH);
      else if (OW >= 2)
        hipLaunchKernelGGL((k_maxpool_bwd_blk<3, 2, true>), grid, dim3(256), 0, stream(), dz, ip,
                           dx, items, H, W, OH, OW, BH, BW, fBW, fBH);
      else
        hipLaunchKernelGGL((k_maxpool_bwd_blk<3, 2, false>), grid, dim3(256), 0, stream(), dz,
                           ip, dx, items, H, W, OH, OW, BH, BW, fBW, fBH);
      return check_launch("maxpool_backward");
    }
    const uint32_t nw = (k + s - 1) / s;
    const dim3 grid(cdiv(xcount, 256));
    const FastDiv fW = make_fastdiv(W), fH = make_fastdiv(H), fS = make_fastdiv(s);
    if (nw == 1)
      hipLaunchKernelGGL(k_maxpool_bwd_gather_n<1>, grid, dim3(256), 0, stream(), dz, ip, dx,
                         xcount, H, W, k, OH, OW, fW, fH, fS);
    else if (nw == 2)
      hipLaunchKernelGGL(k_maxpool_bwd_gather_n<2>, grid, dim3(256), 0, stream(), dz, ip, dx,
                         xcount, H, W, k, OH, OW, fW, fH, fS);
    else if (nw == 3)
      hipLaunchKernelGGL(k_maxpool_bwd_gather_n<3>, grid, dim3(256), 0, stream(), dz, ip, dx,
                         xcount, H, W, k, OH, OW, fW, fH, fS);
    else
      hipLaunchKernelGGL(k_maxpool_bwd_gather, grid, dim3(256), 0, stream(), dz, ip, dx, xcount, H,
                         W, k, s, OH, OW, fW, fH);
    return check_launch("maxpool_backward");
  }
  const uint32_t planes = B * C;
  if (!planes || xcount % planes != 0) {
    set_error("MaxPoolBackwardFused: indices carry no pooling geometry and the input size %u "
              "is not a multiple of batch*channels = %u", xcount, planes);
    return false;
  }
  const uint32_t inPer = xcount / planes;
  if (n == 0) return fill_zero(dx, xcount);
  if (inPer <= kPlaneLds) {
    hipLaunchKernelGGL(k_maxpool_bwd_plane_lds, dim3(planes), dim3(256), inPer * sizeof(float),
                       stream(), dz, ip, dx, OH * OW, inPer);
    return check_launch("maxpool_backward");
  }
  if (!fill_zero(dx, xcount)) return false;
  hipLaunchKernelGGL(k_maxpool_bwd_planes, dim3(cdiv(planes, 64)), dim3(64), 0, stream(), dz, ip,
                     dx, planes, OH * OW, inPer);
  return check_launch("maxpool_backward");
}

// Only the padded-grid layout: G in NCHW order, written by the same plane-
// ordered waves as dx.  An NHWC form (32 channels x 8 blocks per workgroup,
// G through an LDS transpose) measured slower than the plain backward plus
// the conv's own masking pass (AlexNet pool2 76 us against 21 + 22 us): a
// wave's loads and dx stores then span 8 planes, 16-24 cache lines per
// instruction instead of 2-4.
bool maxpool_backward_g_ok(uint32_t C, uint32_t H, uint32_t W, uint32_t OH, uint32_t OW,
                           uint32_t k, uint32_t s, uint32_t layout) {
  return s == 2 && (k == 2 || k == 3) && C && H && W && OH && OW && layout == kGLayoutPad;
}

uint32_t maxpool_backward_g_rows(uint32_t B, uint32_t H, uint32_t W, uint32_t layout) {
  (void)layout;
  return B * cdiv(cdiv(H, 2) * cdiv(W, 2), 64);
}

bool maxpool_backward_g(const float* dz, const float* idx, const float* pooled, float* dx,
                        float* g, float* db, uint32_t B, uint32_t C, uint32_t OH, uint32_t OW,
                        uint32_t H, uint32_t W, uint32_t k, uint32_t layout, uint32_t gw) {
  const uint32_t n = B * C * OH * OW, xcount = B * C * H * W;
  ProfScope prof("maxpool_bwd", 0, 12.0 * n + 4.0 * xcount + 4.0 * double(B) * C * H * gw);
  const uint32_t* ip = reinterpret_cast<const uint32_t*>(idx);
  const uint32_t BW = cdiv(W, 2), nblk = cdiv(H, 2) * BW;
  const FastDiv fBW = make_fastdiv(BW);
  if (layout != kGLayoutPad) {
    set_error("maxpool_backward_g: unsupported G layout %u", layout);
    return false;
  }
  const uint32_t nch = cdiv(nblk, 64), waves = B * C * nch;
  const dim3 grid(cdiv(waves, 4));
  const FastDiv fN = make_fastdiv(nch);
#define DCE_GPAD(K, P)                                                                          \
  hipLaunchKernelGGL((k_maxpool_bwd_gpad<K, P>), grid, dim3(256), 0, stream(), dz, ip, pooled, \
                     dx, g, db, C, H, W, OH, OW, gw, BW, nblk, nch, B, waves, fBW, fN)
  if (k == 2) DCE_GPAD(2, false);
  else if (k == 3 && OW >= 2) DCE_GPAD(3, true);
  else DCE_GPAD(3, false);
#undef DCE_GPAD
  return check_launch("maxpool_backward_g");
}

static bool sh_maxpool_forward(const Dispatch& d) {
  uint32_t B = CU(d, 0), C = CU(d, 1), H = CU(d, 2), W = CU(d, 3), k = CU(d, 4), s = CU(d, 5),
           OH = CU(d, 6), OW = CU(d, 7);
  uint64_t n = uint64_t(B) * C * OH * OW;
  if (!n) return true;
  hipLaunchKernelGGL(k_maxpool_fwd, dim3(cdiv(n, 256)), dim3(256), 0, stream(), S(d, 0), U(d, 0),
                     U(d, 1), B * C, H, W, k, s, OH, OW);
  if (!check_launch("maxpool_forward")) return false;
  // The indices record their window geometry, as those of MaxPoolForwardFused
  // do, so that MaxPoolBackwardFused can run its gather kernels on them.  The
  // geometry must be the one the kernel's output grid implies.
  Buf ib = U(d, 1);
  if (ib.p && uint64_t(ib.n) >= n && k && s && H >= k && W >= k && (H - k) / s + 1 == OH &&
      (W - k) / s + 1 == OW) {
    Buffer* I = static_cast<Buffer*>(d.uavs[1]);
    I->tag = kPoolTag;
    I->meta[0] = H;
    I->meta[1] = W;
    I->meta[2] = k;
    I->meta[3] = s;
  }
  return true;
}
// RunShader("maxpool_backward") keeps the reference's store semantics
// (nn_maxpool_backward.hlsl:21-24): dX[idx] = dZ, the caller clears dX.
__global__ void k_maxpool_bwd_store(Buf dz, Buf idx, Buf dx, uint32_t n) {
  const uint32_t o = gtid();
  if (o >= n) return;
  const uint32_t t = __float_as_uint(ld(idx, o));
  if (t != 0xFFFFFFFFu) st(dx, t, ld(dz, o));
}
static bool sh_maxpool_backward(const Dispatch& d) {
  uint64_t n = uint64_t(CU(d, 0)) * CU(d, 1) * CU(d, 2) * CU(d, 3);
  if (!n) return true;
  hipLaunchKernelGGL(k_maxpool_bwd_store, dim3(cdiv(n, 256)), dim3(256), 0, stream(), S(d, 0),
                     S(d, 1), U(d, 0), uint32_t(n));
  return check_launch("maxpool_backward");
}

// ===========================================================================
// Global average pooling, nearest upsampling, channel concat / slice
// ===========================================================================
__global__ void k_gap(Buf in, Buf out, uint32_t S) {
  __shared__ double sh[4];
  const uint32_t nc = blockIdx.x;
  float s = 0.f;
  for (uint32_t i = threadIdx.x; i < S; i += 256) s += ld(in, nc * S + i);
  const double t = block_sum256(s, sh);
  if (threadIdx.x == 0) st(out, nc, float(t) / float(S));
}
static bool sh_gap(const Dispatch& d) {
  uint32_t BC = CU(d, 0) * CU(d, 1), Sz = CU(d, 2);
  if (!BC || !Sz) return true;
  hipLaunchKernelGGL(k_gap, dim3(BC), dim3(256), 0, stream(), S(d, 0), U(d, 0), Sz);
  return check_launch("global_avg_pool");
}
__global__ void k_gap_bwd(Buf g, Buf dx, uint32_t total, uint32_t S) {
  const uint32_t i = gtid();
  if (i < total) st(dx, i, ld(g, i / S) / float(S));
}
// Quad form (S % 4 == 0, buffers covering the shapes): one g value per quad.
template <bool NT>
__global__ void k_gap_bwd4(const float* __restrict__ g, float* __restrict__ dx, uint32_t total4,
                           FastDiv dS4, float S) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= total4) return;
  const float v = g[fdiv(i, dS4)] / S;
  st4s<NT>(dx + size_t(i) * 4, f4{v, v, v, v});
}
static bool sh_gap_bwd(const Dispatch& d) {
  uint32_t Sz = CU(d, 2);
  uint64_t total = uint64_t(CU(d, 0)) * CU(d, 1) * Sz;
  if (!total) return true;
  ProfScope prof("gap_bwd", 0, 4.0 * double(total));
  const Buf g = S(d, 0), dx = U(d, 0);
  if (Sz % 4 == 0 && total < (1ull << 31) && covers(g, total / Sz) && covers(dx, total) &&
      (reinterpret_cast<uintptr_t>(dx.p) & 15) == 0) {
    const uint32_t total4 = uint32_t(total / 4);
    if (stream_nt(4.0 * double(total)))
      hipLaunchKernelGGL(k_gap_bwd4<true>, dim3(cdiv(total4, 256)), dim3(256), 0, stream(), g.p,
                         dx.p, total4, make_fastdiv(Sz / 4), float(Sz));
    else
      hipLaunchKernelGGL(k_gap_bwd4<false>, dim3(cdiv(total4, 256)), dim3(256), 0, stream(), g.p,
                         dx.p, total4, make_fastdiv(Sz / 4), float(Sz));
    return check_launch("global_avg_pool_backward");
  }
  hipLaunchKernelGGL(k_gap_bwd, dim3(cdiv(total, 256)), dim3(256), 0, stream(), S(d, 0), U(d, 0),
                     uint32_t(total), Sz);
  return check_launch("global_avg_pool_backward");
}

__global__ void k_upsample(Buf X, Buf O, uint32_t total, uint32_t C, uint32_t H, uint32_t W,
                           uint32_t OH, uint32_t OW, uint32_t sH, uint32_t sW) {
  const uint32_t i = gtid();
  if (i >= total) return;
  const uint32_t wo = i % OW, t = i / OW, ho = t % OH, bc = t / OH;
  st(O, i, ld(X, (bc * H + ho / sH) * W + wo / sW));
}
__global__ void k_upsample_bwd(Buf DY, Buf DX, uint32_t total, uint32_t H, uint32_t W,
                               uint32_t OH, uint32_t OW, uint32_t sH, uint32_t sW) {
  const uint32_t i = gtid();
  if (i >= total) return;
  const uint32_t wi = i % W, t = i / W, hi = t % H, bc = t / H;
  float s = 0.f;
  for (uint32_t a = 0; a < sH; ++a) {
    const uint32_t ho = hi * sH + a;
    for (uint32_t b = 0; b < sW; ++b) {
      const uint32_t wo = wi * sW + b;
      if (ho < OH && wo < OW) s += ld(DY, (bc * OH + ho) * OW + wo);
    }
  }
  st(DX, i, s);
}
// Nearest x2 with even W and exact output size: a thread reads an input
// pair (8 bytes) and writes the 2 x 4 outputs it covers as two 16-byte
// stores (output rows 2h and 2h + 1 of plane bc start at 2*row*OW, row =
// bc*H + h).
template <bool NT>
__global__ void k_upsample2(const float* __restrict__ x, float* __restrict__ y, uint32_t pairs,
                            uint32_t W2, FastDiv dW2) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= pairs) return;
  const uint32_t row = fdiv(i, dW2), j = i - row * W2;
  const f2 v = reinterpret_cast<const f2*>(x)[i];
  const f4 q = {v[0], v[0], v[1], v[1]};
  float* o = y + size_t(2 * row) * (4 * W2) + 4 * j;
  st4s<NT>(o, q);
  st4s<NT>(o + 4 * W2, q);
}
static bool sh_upsample(const Dispatch& d) {
  uint32_t B = CU(d, 0), C = CU(d, 1), H = CU(d, 2), W = CU(d, 3), OH = CU(d, 4), OW = CU(d, 5),
           sH = CU(d, 6), sW = CU(d, 7);
  uint64_t total = uint64_t(B) * C * OH * OW;
  if (!total || !sH || !sW) return true;
  ProfScope prof("upsample", 0, 5.0 * double(total));
  const Buf x = S(d, 0), y = U(d, 0);
  const uint64_t nin = uint64_t(B) * C * H * W;
  if (sH == 2 && sW == 2 && OH == 2 * H && OW == 2 * W && W % 2 == 0 && covers(x, nin) &&
      covers(y, total) && (reinterpret_cast<uintptr_t>(x.p) & 7) == 0 &&
      (reinterpret_cast<uintptr_t>(y.p) & 15) == 0 && total < (1ull << 32)) {
    const uint32_t pairs = uint32_t(nin / 2), W2 = W / 2;
    if (stream_nt(5.0 * double(total)))
      hipLaunchKernelGGL(k_upsample2<true>, dim3(cdiv(pairs, 256)), dim3(256), 0, stream(), x.p,
                         y.p, pairs, W2, make_fastdiv(W2));
    else
      hipLaunchKernelGGL(k_upsample2<false>, dim3(cdiv(pairs, 256)), dim3(256), 0, stream(), x.p,
                         y.p, pairs, W2, make_fastdiv(W2));
    return check_launch("upsample");
  }
  hipLaunchKernelGGL(k_upsample, dim3(cdiv(total, 256)), dim3(256), 0, stream(), S(d, 0),
                     U(d, 0), uint32_t(total), C, H, W, OH, OW, sH, sW);
  return check_launch("upsample");
}
// Nearest x2 with even W and exact output size: a thread sums two 2 x 2
// blocks (two quads of dy rows 2h and 2h+1) into a pair of dx values, in the
// reference's (a, then b) order.
template <bool NT>
__global__ void k_upsample2_bwd(const float* __restrict__ dy, float* __restrict__ dx,
                                uint32_t pairs, uint32_t W2, FastDiv dW2) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= pairs) return;
  const uint32_t row = fdiv(i, dW2), j = i - row * W2;  // row = bc*H + h
  const f4 a = ld4s<NT>(dy + (size_t(2 * row) * W2 + j) * 4);
  const f4 b = ld4s<NT>(dy + (size_t(2 * row + 1) * W2 + j) * 4);
  reinterpret_cast<f2*>(dx)[i] = f2{((a[0] + a[1]) + b[0]) + b[1], ((a[2] + a[3]) + b[2]) + b[3]};
}
static bool sh_upsample_bwd(const Dispatch& d) {
  uint32_t B = CU(d, 0), C = CU(d, 1), H = CU(d, 2), W = CU(d, 3), OH = CU(d, 4), OW = CU(d, 5),
           sH = CU(d, 6), sW = CU(d, 7);
  uint64_t total = uint64_t(B) * C * H * W;
  if (!total) return true;
  ProfScope prof("upsample_bwd", 0, 4.0 * double(total) + 4.0 * double(B) * C * OH * OW);
  const Buf dyb = S(d, 0), dxb = U(d, 0);
  if (sH == 2 && sW == 2 && OH == 2 * H && OW == 2 * W && W % 2 == 0 && 4 * total < (1ull << 31) &&
      covers(dyb, 4 * total) && covers(dxb, total) &&
      ((reinterpret_cast<uintptr_t>(dyb.p) | reinterpret_cast<uintptr_t>(dxb.p)) & 15) == 0) {
    const uint32_t pairs = uint32_t(total / 2), W2 = W / 2;
    if (stream_nt(20.0 * double(total)))
      hipLaunchKernelGGL(k_upsample2_bwd<true>, dim3(cdiv(pairs, 256)), dim3(256), 0, stream(),
                         dyb.p, dxb.p, pairs, W2, make_fastdiv(W2));
    else
      hipLaunchKernelGGL(k_upsample2_bwd<false>, dim3(cdiv(pairs, 256)), dim3(256), 0, stream(),
                         dyb.p, dxb.p, pairs, W2, make_fastdiv(W2));
    return check_launch("upsample_backward");
  }
  hipLaunchKernelGGL(k_upsample_bwd, dim3(cdiv(total, 256)), dim3(256), 0, stream(), S(d, 0),
                     U(d, 0), uint32_t(total), H, W, OH, OW, sH, sW);
  return check_launch("upsample_backward");
}

// MODE 0: concat_insert (Out[b, c+off, s] = X[b, c, s]); MODE 1: slice (DX[b, c, s] = DY[b, c+off, s])
template <int MODE>
__global__ void k_chan_copy(Buf src, Buf dst, uint32_t total, uint32_t cin, uint32_t S,
                            uint32_t cout, uint32_t coff) {
  const uint32_t i = gtid();
  if (i >= total) return;
  const uint32_t s = i % S, t = i / S, c = t % cin, b = t / cin;
  const uint32_t o = (b * cout + c + coff) * S + s;
  if (MODE == 0)
    st(dst, o, ld(src, i));
  else
    st(dst, i, ld(src, o));
}
// Quad form (S % 4 == 0, buffers covering the shapes, 16-byte aligned).
template <int MODE, bool NT>
__global__ void k_chan_copy4(const float* __restrict__ src, float* __restrict__ dst,
                             uint32_t total4, uint32_t cin, uint32_t S4, uint32_t cout,
                             uint32_t coff, FastDiv dS4, FastDiv dCin) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= total4) return;
  const uint32_t t = fdiv(i, dS4), s4 = i - t * S4;
  const uint32_t b = fdiv(t, dCin), c = t - b * cin;
  const uint32_t o = (b * cout + c + coff) * S4 + s4;
  if (MODE == 0)
    st4s<NT>(dst + size_t(o) * 4, ld4s<NT>(src + size_t(i) * 4));
  else
    st4s<NT>(dst + size_t(i) * 4, ld4s<NT>(src + size_t(o) * 4));
}
template <int MODE>
static bool sh_chan_copy(const Dispatch& d) {
  uint32_t B = CU(d, 0), cin = CU(d, 1), Sz = CU(d, 2), cout = CU(d, 3), coff = CU(d, 4);
  uint64_t total = uint64_t(B) * cin * Sz;
  if (!total) return true;
  ProfScope prof(MODE == 0 ? "concat_insert" : "slice", 0, 8.0 * double(total));
  {
    const Buf src = S(d, 0), dst = U(d, 0);
    const uint64_t big = uint64_t(B) * cout * Sz;  // the concatenated tensor
    if (Sz % 4 == 0 && cin + coff <= cout && big < (1ull << 31) &&
        covers(MODE == 0 ? src : dst, total) && covers(MODE == 0 ? dst : src, big) &&
        ((reinterpret_cast<uintptr_t>(src.p) | reinterpret_cast<uintptr_t>(dst.p)) & 15) == 0) {
      const uint32_t total4 = uint32_t(total / 4);
      if (stream_nt(8.0 * double(total)))
        hipLaunchKernelGGL((k_chan_copy4<MODE, true>), dim3(cdiv(total4, 256)), dim3(256), 0,
                           stream(), src.p, dst.p, total4, cin, Sz / 4, cout, coff,
                           make_fastdiv(Sz / 4), make_fastdiv(cin));
      else
        hipLaunchKernelGGL((k_chan_copy4<MODE, false>), dim3(cdiv(total4, 256)), dim3(256), 0,
                           stream(), src.p, dst.p, total4, cin, Sz / 4, cout, coff,
                           make_fastdiv(Sz / 4), make_fastdiv(cin));
      return check_launch(MODE == 0 ? "concat_insert" : "slice");
    }
  }
  hipLaunchKernelGGL(k_chan_copy<MODE>, dim3(cdiv(total, 256)), dim3(256), 0, stream(), S(d, 0),
                     U(d, 0), uint32_t(total), cin, Sz, cout, coff);
  return check_launch(MODE == 0 ? "concat_insert" : "slice");
}

// ===========================================================================
// Depthwise convolution (filters (C,1,kH,kW), bias (C))
// ===========================================================================
struct DwGeom {
  uint32_t B, C, H, W, kH, kW, s, p, OH, OW;
};
static DwGeom dw_geom(const Dispatch& d) {
  DwGeom g{CU(d, 0), CU(d, 1), CU(d, 2), CU(d, 3), CU(d, 4), CU(d, 5), CU(d, 6), CU(d, 7), CU(d, 8), 0};
  // nn_depthwise_conv_*.hlsl recompute OW from the other constants.
  g.OW = (g.s && g.W + 2 * g.p >= g.kW) ? (g.W + 2 * g.p - g.kW) / g.s + 1 : 0;
  return g;
}
__global__ void k_dw_fwd(Buf x, Buf f, Buf bias, Buf y, DwGeom g, uint32_t total) {
  const uint32_t i = gtid();
  if (i >= total) return;
  const uint32_t ow = i % g.OW, t = i / g.OW, oh = t % g.OH, t2 = t / g.OH, c = t2 % g.C;
  const uint32_t n = t2 / g.C;
  const uint32_t xb = (n * g.C + c) * g.H * g.W, fb = c * g.kH * g.kW;
  float s = 0.f;
  for (uint32_t fh = 0; fh < g.kH; ++fh) {
    const int ih = int(oh * g.s + fh) - int(g.p);
    if (ih < 0 || ih >= int(g.H)) continue;
    for (uint32_t fw = 0; fw < g.kW; ++fw) {
      const int iw = int(ow * g.s + fw) - int(g.p);
      if (iw < 0 || iw >= int(g.W)) continue;
      s += ld(x, xb + uint32_t(ih) * g.W + uint32_t(iw)) * ld(f, fb + fh * g.kW + fw);
    }
  }
  st(y, i, s + ld(bias, c));
}
__global__ void k_dw_bwd_input(Buf dy, Buf f, Buf dx, DwGeom g, uint32_t total) {
  const uint32_t i = gtid();
  if (i >= total) return;
  const uint32_t iw = i % g.W, t = i / g.W, ih = t % g.H, t2 = t / g.H, c = t2 % g.C;
  const uint32_t n = t2 / g.C;
  const uint32_t gb = (n * g.C + c) * g.OH * g.OW, fb = c * g.kH * g.kW;
  float s = 0.f;
  for (uint32_t fh = 0; fh < g.kH; ++fh) {
    const int ohs = int(ih) - int(fh) + int(g.p);
    if (ohs < 0 || ohs % int(g.s) != 0) continue;
    const uint32_t oh = uint32_t(ohs) / g.s;
    if (oh >= g.OH) continue;
    for (uint32_t fw = 0; fw < g.kW; ++fw) {
      const int ows = int(iw) - int(fw) + int(g.p);
      if (ows < 0 || ows % int(g.s) != 0) continue;
      const uint32_t ow = uint32_t(ows) / g.s;
      if (ow >= g.OW) continue;
      s += ld(dy, gb + oh * g.OW + ow) * ld(f, fb + fh * g.kW + fw);
    }
  }
  st(dx, i, s);
}
// One pass over dy per (channel, piece): every thread keeps all kH*kW+1
// running sums (df taps and db) for the outputs it visits.
constexpr int kDwMaxTaps = 25;
__global__ void k_dw_bwd_filter_part(Buf dy, Buf x, DwGeom g, uint32_t pieces, double* part) {
  __shared__ double sh[4];
  const uint32_t c = blockIdx.y, pc = blockIdx.x;
  const uint32_t taps = g.kH * g.kW;
  const uint32_t len = g.B * g.OH * g.OW;
  const uint32_t i0 = uint32_t((uint64_t(len) * pc) / pieces);
  const uint32_t i1 = uint32_t((uint64_t(len) * (pc + 1)) / pieces);
  float acc[kDwMaxTaps + 1];
#pragma unroll
  for (int t = 0; t <= kDwMaxTaps; ++t) acc[t] = 0.f;
  const uint32_t ohw = g.OH * g.OW;
  for (uint32_t i = i0 + threadIdx.x; i < i1; i += 256) {
    const uint32_t n = i / ohw, r = i - n * ohw, oh = r / g.OW, ow = r - oh * g.OW;
    const float gv = ld(dy, (n * g.C + c) * ohw + r);
    acc[kDwMaxTaps] += gv;
    const uint32_t xb = (n * g.C + c) * g.H * g.W;
#pragma unroll
    for (int t = 0; t < kDwMaxTaps; ++t) {
      if (uint32_t(t) < taps) {
        const uint32_t fh = uint32_t(t) / g.kW, fw = uint32_t(t) - fh * g.kW;
        const int ih = int(oh * g.s + fh) - int(g.p);
        const int iw = int(ow * g.s + fw) - int(g.p);
        float xv = 0.f;
        if (ih >= 0 && ih < int(g.H) && iw >= 0 && iw < int(g.W))
          xv = ld(x, xb + uint32_t(ih) * g.W + uint32_t(iw));
        acc[t] += gv * xv;
      }
    }
  }
  // Static indices keep acc[] in registers; the condition is block-uniform.
#pragma unroll
  for (int t = 0; t <= kDwMaxTaps; ++t) {
    if (uint32_t(t) < taps || t == kDwMaxTaps) {
      const double s = block_sum256(acc[t], sh);
      const uint32_t slot = (t == kDwMaxTaps) ? taps : uint32_t(t);
      if (threadIdx.x == 0) part[(size_t(c) * pieces + pc) * (taps + 1) + slot] = s;
    }
  }
}
// One wave per output (c, t): lane l adds pieces l, l+64, ..., then a DPP
// wave reduction.  Four outputs per 256 threads.
__global__ void __launch_bounds__(256)
    k_dw_bwd_filter_final(const double* part, uint32_t pieces, uint32_t C, uint32_t taps, Buf df,
                          Buf db) {
  const uint32_t i = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (i >= C * (taps + 1)) return;  // whole waves leave together
  const uint32_t c = i / (taps + 1), t = i - c * (taps + 1);
  double a = 0;
  for (uint32_t p = lane; p < pieces; p += 64) a += part[(size_t(c) * pieces + p) * (taps + 1) + t];
  const double s = wave_reduce(a);
  if (lane != 0) return;
  if (t == taps)
    st(db, c, float(s));
  else
    st(df, c * taps + t, float(s));
}
// Pipelined band kernels for the common shapes (K x K taps with K in {3, 5},
// stride S in {1, 2}, pad < K, natural output size).  A block walks a list of
// bands (rows of one (image, channel) plane).  A band's input window (zero
// outside the plane) is loaded into registers -- at most kDwRegs values per
// thread, through a buffer resource so that out-of-plane reads return zero
// with no branch -- then written to LDS; the next band's loads are issued
// before the current band is computed, so global traffic overlaps the
// stencil work.  Each thread computes a 2 x 2 block of outputs from one
// register window read out of LDS.
constexpr int kDwRegs = 16;
constexpr uint32_t kDwBand = 256 * kDwRegs;  // LDS floats one band window may use

// A window of R rows x LW columns of a rows x cols plane, anchored at plane
// row rb / column cb (either may be negative); cells outside the plane are 0.
struct DwWin {
  int rb, cb;
  uint32_t R, LW;
};
template <int N>
__device__ __forceinline__ void dw_win_load(const BRes& b, uint32_t base, uint32_t rows,
                                            uint32_t cols, const DwWin& w, FastDiv dLW,
                                            float (&v)[N]) {
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const uint32_t e = u * 256 + threadIdx.x;
    const uint32_t i = fdiv(e, dLW), j = e - i * w.LW;
    const int r = w.rb + int(i), c = w.cb + int(j);
    const bool ok = e < w.R * w.LW && r >= 0 && r < int(rows) && c >= 0 && c < int(cols);
    v[u] = b.ld1(ok ? base + uint32_t(r) * cols + uint32_t(c) : kOob);
  }
}
template <int N>
__device__ __forceinline__ void dw_win_store(float* lds, const float (&v)[N], uint32_t n) {
#pragma unroll
  for (int u = 0; u < N; ++u)
    if (u * 256 + threadIdx.x < n) lds[u * 256 + threadIdx.x] = v[u];
}
// Quad form, for planes whose width is a multiple of 4: the stored window
// starts lo = cb & 3 columns left of the logical one, at a 4-aligned plane
// column, and its width w.LW (the stored width) is a multiple of 4.  Each
// quad then lies wholly inside or wholly outside the plane and is one 16-byte
// buffer load (a quarter of the loads and index divisions of the dword form).
template <int N, bool NT = false>
__device__ __forceinline__ void dw_win_load4(const BRes& b, uint32_t base, uint32_t rows,
                                             uint32_t cols, const DwWin& w, FastDiv dQW,
                                             f4 (&v)[N]) {
  const int cs = w.cb - (w.cb & 3);
  const uint32_t qw = w.LW / 4;
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const uint32_t q = u * 256 + threadIdx.x;
    const uint32_t i = fdiv(q, dQW), jq = q - i * qw;
    const int r = w.rb + int(i), c = cs + 4 * int(jq);
    const bool ok = q < w.R * qw && r >= 0 && r < int(rows) && c >= 0 && c < int(cols);
    const uint32_t off = ok ? base + uint32_t(r) * cols + uint32_t(c) : kOob;
    v[u] = NT ? b.ld4nt(off) : b.ld4(off);
  }
}
template <int N>
__device__ __forceinline__ void dw_win_store4(float* lds, const f4 (&v)[N], uint32_t nq) {
#pragma unroll
  for (int u = 0; u < N; ++u)
    if (u * 256 + threadIdx.x < nq) *reinterpret_cast<f4*>(lds + 4 * (u * 256 + threadIdx.x)) = v[u];
}
// A band window in dword or quad form (V4), with the quad form's column shift.
template <bool V4, int N>
struct DwRegs {
  float v[V4 ? 1 : N];
  f4 q[V4 ? N / 4 : 1];
  // NT: nontemporal quad loads (the dword form has no such variant).
  template <bool NT = false>
  __device__ __forceinline__ void load(const BRes& b, uint32_t base, uint32_t rows, uint32_t cols,
                                       const DwWin& w, FastDiv d) {
    if constexpr (V4)
      dw_win_load4<N / 4, NT>(b, base, rows, cols, w, d, q);
    else
      dw_win_load(b, base, rows, cols, w, d, v);
  }
  __device__ __forceinline__ void store(float* lds, uint32_t R, uint32_t LW) const {
    if constexpr (V4)
      dw_win_store4(lds, q, R * LW / 4);
    else
      dw_win_store(lds, v, R * LW);
  }
  // Stored column of logical window column 0.
  __device__ static __forceinline__ int shift(int cb) { return V4 ? (cb & 3) : 0; }
  // Phase-split store: stored column j of a row goes to (j % P) * (LW / P) +
  // j / P (LW % P == 0), so lanes reading columns P apart hit consecutive
  // LDS words instead of every P-th bank.  d divides by LW / 4 (V4) or LW.
  template <int P>
  __device__ __forceinline__ void store_ph(float* lds, uint32_t R, uint32_t LW, FastDiv d) const {
    static_assert(P == 2 || P == 4, "phase count");
    const uint32_t LP = LW / P;
    if constexpr (V4) {
      const uint32_t qw = LW / 4;
#pragma unroll
      for (int u = 0; u < N / 4; ++u) {
        const uint32_t qi = u * 256 + threadIdx.x;
        if (qi < R * qw) {
          const uint32_t i = fdiv(qi, d), jq = qi - i * qw;
          float* row = lds + i * LW + (4 / P) * jq;
#pragma unroll
          for (int e = 0; e < 4; ++e) row[(e % P) * LP + e / P] = q[u][e];
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < N; ++u) {
        const uint32_t e = u * 256 + threadIdx.x;
        if (e < R * LW) {
          const uint32_t i = fdiv(e, d), j = e - i * LW;
          lds[i * LW + (j % P) * LP + j / P] = v[u];
        }
      }
    }
  }
};

// Sub-pixel geometry of the stride-2 input gradient: with p = 2*ph + PODD,
// output row 2A + r takes tap fh exactly when r + PODD - fh is even, from dy
// row A + ph + (r + PODD - fh) / 2.  Window row j holds dy row A + ph + JMIN + j.
template <int K, int PODD>
struct DwS2 {
  static constexpr int JMIN = -((K - 1 - PODD + 1) / 2);  // floor((PODD - K + 1) / 2)
  static constexpr int JMAX = (1 + PODD) / 2;
  static constexpr int WR = JMAX - JMIN + 1;
};

// dX band: input rows [r0, r0 + RB) (RB even) of plane (n, c).
//   S = 1: LDS cell (i, j) = dy[r0 + p - (K-1) + i][p - (K-1) + j]; output
//          block (2a, 2b) reads the (K+1) x (K+1) window at (2a, 2b).
//   S = 2: LDS cell (i, j) = dy[r0/2 + ph + JMIN + i][ph + JMIN + j]; output
//          block (2a, 2b) reads the WR x WR window at (a, b).
// A thread takes 2 rows x CW columns (CW / 2 such blocks side by side, one
// register window of WR x WC) and stores each row's CW outputs as one
// vector store when they lie in the row (unaligned for rows whose length is
// not a multiple of CW: unaligned access is on).  Taps are summed in
// (fh, fw) order for every output, as the generic kernel.
template <int K, int S, int PODD, bool V4, int CW, bool NT>
__global__ void __launch_bounds__(256)
    k_dw_bwd_input_band(const float* __restrict__ dy, const float* __restrict__ f,
                        float* __restrict__ dx, uint32_t C, uint32_t H, uint32_t W, uint32_t OH,
                        uint32_t OW, uint32_t p, uint32_t RB, uint32_t nb, uint32_t nbands,
                        uint32_t LR, uint32_t LW, uint32_t BW, uint32_t ndy, FastDiv dLW,
                        FastDiv dNb, FastDiv dBW) {
  static_assert(CW == 2 || CW == 4, "2 or 4 columns per thread");
  constexpr int WR = S == 1 ? K + 1 : DwS2<K, PODD>::WR;
  constexpr int WC = S == 1 ? WR + CW - 2 : WR + CW / 2 - 1;
  __shared__ __attribute__((aligned(16))) float sd[kDwBand];
  BRes bd;
  bd.init(dy, ndy);
  DwRegs<V4, kDwRegs> v;
  const uint32_t ph = p / 2;
  auto decode = [&](uint32_t band, uint32_t& plane, uint32_t& r0) {
    plane = fdiv(band, dNb);
    r0 = (band - plane * nb) * RB;
  };
  auto win = [&](uint32_t r0) {
    DwWin w;
    w.R = LR;
    w.LW = LW;
    if (S == 1) {
      w.rb = int(r0) + int(p) - (K - 1);
      w.cb = int(p) - (K - 1);
    } else {
      w.rb = int(r0 / 2 + ph) + DwS2<K, PODD>::JMIN;
      w.cb = int(ph) + DwS2<K, PODD>::JMIN;
    }
    return w;
  };
  const int lo = DwRegs<V4, kDwRegs>::shift(win(0).cb);
  uint32_t band = blockIdx.x;
  if (band < nbands) {
    uint32_t plane, r0;
    decode(band, plane, r0);
    v.load(bd, plane * OH * OW, OH, OW, win(r0), dLW);
  }
  for (; band < nbands; band += gridDim.x) {
    uint32_t plane, r0;
    decode(band, plane, r0);
    const uint32_t c = plane % C;
    __syncthreads();  // the previous band's LDS reads are done
    v.store(sd, LR, LW);
    __syncthreads();
    if (band + gridDim.x < nbands) {
      uint32_t pn, rn;
      decode(band + gridDim.x, pn, rn);
      v.load(bd, pn * OH * OW, OH, OW, win(rn), dLW);
    }
    float w[K * K];
#pragma unroll
    for (int t = 0; t < K * K; ++t) w[t] = f[c * K * K + t];
    const uint32_t r1 = min(r0 + RB, H);
    float* dxp = dx + size_t(plane) * H * W;
    const uint32_t items = ((r1 - r0 + 1) / 2) * BW;
    for (uint32_t e = threadIdx.x; e < items; e += 256) {
      const uint32_t a = fdiv(e, dBW), q = e - a * BW;
      const uint32_t i0 = S == 1 ? 2 * a : a, j0 = S == 1 ? CW * q : (CW / 2) * q;
      float win_[WR][WC];
#pragma unroll
      for (int i = 0; i < WR; ++i)
#pragma unroll
        for (int j = 0; j < WC; ++j) win_[i][j] = sd[(i0 + i) * LW + j0 + j + lo];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const uint32_t ih = r0 + 2 * a + r;
        float o[CW];
#pragma unroll
        for (int cc = 0; cc < CW; ++cc) {
          // Column c2 of 2x2 block sb, whose window starts co columns in.
          const int sb = cc / 2, c2 = cc % 2, co = S == 1 ? 2 * sb : sb;
          float acc = 0.f;
#pragma unroll
          for (int fh = 0; fh < K; ++fh) {
#pragma unroll
            for (int fw = 0; fw < K; ++fw) {
              if (S == 1) {
                acc += win_[r + K - 1 - fh][co + c2 + K - 1 - fw] * w[fh * K + fw];
              } else if (((r + PODD - fh) & 1) == 0 && ((c2 + PODD - fw) & 1) == 0) {
                constexpr int J = DwS2<K, PODD>::JMIN;
                acc += win_[(r + PODD - fh) / 2 - J][co + (c2 + PODD - fw) / 2 - J] * w[fh * K + fw];
              }
            }
          }
          o[cc] = acc;
        }
        if (ih < r1) {
          const uint32_t col = CW * q;
          float* row = dxp + size_t(ih) * W + col;
          if (col + CW - 1 < W) {
            if constexpr (CW == 4 && NT) {
              // Rows of a multiple of 4 floats keep the quads 16-byte aligned.
              if ((W & 3) == 0)
                stnt4(row, f4{o[0], o[1], o[2], o[3]});
              else
                stu(row, f4{o[0], o[1], o[2], o[3]});
            } else if constexpr (CW == 4)
              stu(row, f4{o[0], o[1], o[2], o[3]});
            else
              stu(row, f2{o[0], o[1]});
          } else {
#pragma unroll
            for (int cc = 0; cc < CW; ++cc)
              if (col + cc < W) row[cc] = o[cc];
          }
        }
      }
    }
  }
}

// Forward band: output rows [o0, o0 + RB) (RB even) of plane (n, c).  LDS
// cell (i, j) = x[o0*S - p + i][j - p] (window R x LW, zero outside the
// plane); output block (2a, 2b) reads the (S + K) x (S + K) window at
// (2a*S, 2b*S).  Taps are summed in (fh, fw) order and the bias added last,
// as in the generic kernel.  An output pair inside its row is one 8-byte
// store (4-byte aligned for rows of odd length: unaligned access is on).
// STATS: the band also leaves the batch-norm statistics of what it stores,
// the double sums of y and y*y (threads add their values in float, then
// the block tree in double) at stats[(c * B * nb + n * nb + band) * 2]:
// one piece per band of each image, [C][B * nb][2].
template <int K, int S, bool V4, bool STATS>
__global__ void __launch_bounds__(256)
    k_dw_fwd_band(const float* __restrict__ x, const float* __restrict__ f,
                  const float* __restrict__ bias, float* __restrict__ y, uint32_t C, uint32_t H,
                  uint32_t W, uint32_t OH, uint32_t OW, uint32_t p, uint32_t RB, uint32_t nb,
                  uint32_t nbands, uint32_t LR, uint32_t LW, uint32_t BW, uint32_t nx,
                  FastDiv dLW, FastDiv dNb, FastDiv dBW, double* __restrict__ stats) {
  constexpr int XW = S + K;
  __shared__ __attribute__((aligned(16))) float sd[kDwBand];
  __shared__ double ssum[4];
  BRes bx;
  bx.init(x, nx);
  DwRegs<V4, kDwRegs> v;
  auto decode = [&](uint32_t band, uint32_t& plane, uint32_t& o0) {
    plane = fdiv(band, dNb);
    o0 = (band - plane * nb) * RB;
  };
  auto win = [&](uint32_t o0) {
    DwWin w;
    w.R = LR;
    w.LW = LW;
    w.rb = int(o0 * S) - int(p);
    w.cb = -int(p);
    return w;
  };
  const int lo = DwRegs<V4, kDwRegs>::shift(win(0).cb);
  uint32_t band = blockIdx.x;
  if (band < nbands) {
    uint32_t plane, o0;
    decode(band, plane, o0);
    v.load(bx, plane * H * W, H, W, win(o0), dLW);
  }
  for (; band < nbands; band += gridDim.x) {
    uint32_t plane, o0;
    decode(band, plane, o0);
    const uint32_t c = plane % C;
    __syncthreads();  // the previous band's LDS reads are done
    v.store(sd, LR, LW);
    __syncthreads();
    if (band + gridDim.x < nbands) {
      uint32_t pn, on;
      decode(band + gridDim.x, pn, on);
      v.load(bx, pn * H * W, H, W, win(on), dLW);
    }
    float w[K * K];
#pragma unroll
    for (int t = 0; t < K * K; ++t) w[t] = f[c * K * K + t];
    const float bc = bias[c];
    const uint32_t o1 = min(o0 + RB, OH);
    float* yp = y + size_t(plane) * OH * OW;
    const uint32_t items = ((o1 - o0 + 1) / 2) * BW;
    float f0 = 0.f, f1 = 0.f;
    for (uint32_t e = threadIdx.x; e < items; e += 256) {
      const uint32_t a = fdiv(e, dBW), b2 = e - a * BW;
      float win_[XW][XW];
#pragma unroll
      for (int i = 0; i < XW; ++i)
#pragma unroll
        for (int j = 0; j < XW; ++j) win_[i][j] = sd[(2 * a * S + i) * LW + 2 * b2 * S + j + lo];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const uint32_t oh = o0 + 2 * a + r;
        float o[2];
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          float acc = 0.f;
#pragma unroll
          for (int fh = 0; fh < K; ++fh)
#pragma unroll
            for (int fw = 0; fw < K; ++fw) acc += win_[r * S + fh][cc * S + fw] * w[fh * K + fw];
          o[cc] = acc + bc;
        }
        if (oh < o1) {
          float* row = yp + size_t(oh) * OW + 2 * b2;
          if (2 * b2 + 1 < OW) {
            stu(row, f2{o[0], o[1]});
            if constexpr (STATS) {
              f0 += o[0] + o[1];
              f1 = fmaf(o[1], o[1], fmaf(o[0], o[0], f1));
            }
          } else {
            row[0] = o[0];
            if constexpr (STATS) {
              f0 += o[0];
              f1 = fmaf(o[0], o[0], f1);
            }
          }
        }
      }
    }
    if constexpr (STATS) {
      const double s0 = block_sum256(double(f0), ssum);
      const double s1 = block_sum256(double(f1), ssum);
      if (threadIdx.x == 0) {
        const uint32_t n = plane / C, pieces = (nbands / C);
        double* d = stats + (size_t(c) * pieces + n * nb + (band - plane * nb)) * 2;
        d[0] = s0;
        d[1] = s1;
      }
    }
  }
}

// LDS floats of the filter kernels' dy band window: a full band for stride 1
// (bands of up to 73 rows at 56 wide: one band per 56x56 image, 52 -> 47 us
// at MobileNetV2's s1 shape), half of one for stride 2 (the larger x window
// is the limit there, and more LDS per block cost occupancy: 73 -> 77 us).
__host__ __device__ constexpr uint32_t dw_gband(uint32_t S) { return S == 1 ? kDwBand : kDwBand / 2; }

// dW / db partials.  Block (c, piece) walks a contiguous range of channel c's
// B * nb units (unit u = band u mod nb of image u / nb: output rows
// [o0, o0 + RB), RB even); the ranges split the units evenly over the pieces:
//   LDS x cell (i, j) = x[o0*S - p + i][j - p]      (LXR x LXW, zero outside)
//   LDS g cell (i, j) = dy[o0 + i][j]               (LGR x LGW, zero outside; S = 2)
// A thread takes 2 x 2 blocks of dy (items e = tid + 256 i of the band's
// (LGR / 2) x (LGW / 2) blocks) and the (S + K) x (S + K) x window under them.
// Stride 1: each dy value is used by one thread only, so the thread loads its
// blocks (at most NI) straight into registers -- the next unit's while the
// current one is multiplied, zero outside the plane -- and only the x window,
// which neighbouring blocks share, goes through LDS (64x144x56x56: 44.3 ->
// 41.9 us).  Stride 2 stages the dy window in LDS too (the register form
// measured 68 -> 75 us at 64x96x112x112).  NT: nontemporal loads, for
// passes larger than the MALL (stride 2 at 64x96x112x112: 68 -> 63 us).  The
// K*K + 1 running sums are reduced once per block (waves by shuffle, then
// the 4 wave sums in order) and stored as part[c][piece][t] (double).
template <int K, int S, bool V4, bool NT>
__global__ void __launch_bounds__(256)
    k_dw_bwd_filter_band(const float* __restrict__ dy, const float* __restrict__ x,
                         double* __restrict__ part, uint32_t B, uint32_t C, uint32_t H,
                         uint32_t W, uint32_t OH, uint32_t OW, uint32_t p, uint32_t RB,
                         uint32_t nb, uint32_t LXR, uint32_t LXW, uint32_t LGR, uint32_t LGW,
                         FastDiv dLXW, FastDiv dLGW, FastDiv dNb, FastDiv dBW) {
  constexpr int T = K * K + 1;
  constexpr int XW = S + K;  // x window edge under a 2 x 2 dy block
  constexpr bool GREG = S == 1;                       // dy blocks in registers
  constexpr int NI = GREG ? int(dw_gband(S) / 1024) : 1;  // LGR * LGW <= dw_gband(S)
  __shared__ __attribute__((aligned(16))) float sx[kDwBand];
  __shared__ __attribute__((aligned(16))) float sg[GREG ? 4 : dw_gband(S)];
  __shared__ float red[4][T];
  const uint32_t c = blockIdx.x, piece = blockIdx.y, npieces = gridDim.y;
  BRes bx, bg;
  bx.init(x, B * C * H * W);
  bg.init(dy, B * C * OH * OW);
  DwRegs<V4, kDwRegs> xv;
  DwRegs<V4, GREG ? 4 : dw_gband(S) / 256> gv;  // S = 2: the next unit's dy window
  const int lox = DwRegs<V4, kDwRegs>::shift(-int(p));
  // The channel's B * nb (image, band) units, split evenly over the pieces.
  const uint32_t units = B * nb;
  const uint32_t u0 = uint32_t(uint64_t(units) * piece / npieces);
  const uint32_t total = uint32_t(uint64_t(units) * (piece + 1) / npieces) - u0;
  const uint32_t items = (LGR / 2) * (LGW / 2);
  // Stride 1: this thread's 2 x 2 blocks, band rows 2a, columns 2b (fixed for
  // every unit), and the next unit's dy values of them.
  uint32_t ia[NI], ib[NI];
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const uint32_t e = threadIdx.x + 256u * it;
    ia[it] = fdiv(e, dBW);
    ib[it] = e - ia[it] * (LGW / 2);
  }
  float gq[NI][4];
  auto issue = [&](uint32_t j) {
    const uint32_t u = u0 + j;
    const uint32_t n = fdiv(u, dNb), o0 = (u - n * nb) * RB;
    const uint32_t plane = n * C + c;
    xv.template load<NT>(bx, plane * H * W, H, W, DwWin{int(o0 * S) - int(p), -int(p), LXR, LXW},
                         dLXW);
    if constexpr (!GREG) {
      gv.template load<NT>(bg, plane * OH * OW, OH, OW, DwWin{int(o0), 0, LGR, LGW}, dLGW);
    } else {
      const uint32_t gb = plane * OH * OW;
#pragma unroll
      for (int it = 0; it < NI; ++it) {
        const bool in = threadIdx.x + 256u * it < items;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const uint32_t row = o0 + 2 * ia[it] + r, col = 2 * ib[it];
          if (V4) {
            // Rows of a multiple of 4 floats: the pair is one 8-byte load.
            const uint32_t off = in && row < OH && col < OW ? gb + row * OW + col : kOob;
            const f2 v = NT ? bg.ld2nt(off) : bg.ld2(off);
            gq[it][2 * r] = v[0];
            gq[it][2 * r + 1] = v[1];
          } else {
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
              gq[it][2 * r + cc] =
                  bg.ld1(in && row < OH && col + cc < OW ? gb + row * OW + col + cc : kOob);
          }
        }
      }
    }
  };
  // Stride 2: LDS rows are stored phase-split, x by column mod 4 and dy by
  // column mod 2.  A thread's x columns 4*b2 + jj + lox then sit at b2 +
  // xo[jj] and its dy columns 2*b2 + cc at b2 + cc * LGW / 2, so consecutive
  // lanes (consecutive b2) read consecutive words instead of every 4th bank
  // (s2 dW 77 -> 74 us at MobileNetV2's 112x112).
  constexpr int PX = S == 2 ? 4 : 1, PG = S == 2 ? 2 : 1;
  int xo[XW];
#pragma unroll
  for (int jj = 0; jj < XW; ++jj) xo[jj] = ((jj + lox) % PX) * int(LXW / PX) + (jj + lox) / PX;
  float acc[T];
#pragma unroll
  for (int q = 0; q < T; ++q) acc[q] = 0.f;
  // One 2 x 2 dy block g with the x window under block (a, b2).
  auto block = [&](uint32_t a, uint32_t b2, const float (&g)[2][2]) {
    float xw[XW][XW];
#pragma unroll
    for (int i = 0; i < XW; ++i)
#pragma unroll
      for (int jj = 0; jj < XW; ++jj) xw[i][jj] = sx[(2 * a * S + i) * LXW + (2 * S / PX) * b2 + xo[jj]];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        acc[K * K] += g[r][cc];
#pragma unroll
        for (int fh = 0; fh < K; ++fh)
#pragma unroll
          for (int fw = 0; fw < K; ++fw) acc[fh * K + fw] += g[r][cc] * xw[r * S + fh][cc * S + fw];
      }
  };
  if (total) issue(0);
  for (uint32_t jb = 0; jb < total; ++jb) {
    __syncthreads();  // the previous band's LDS reads are done
    if constexpr (S == 2) {
      xv.template store_ph<PX>(sx, LXR, LXW, dLXW);
      gv.template store_ph<PG>(sg, LGR, LGW, dLGW);
    } else {
      xv.store(sx, LXR, LXW);
    }
    float gc[NI][4];
#pragma unroll
    for (int it = 0; it < NI; ++it)
#pragma unroll
      for (int v = 0; v < 4; ++v) gc[it][v] = gq[it][v];
    __syncthreads();
    if (jb + 1 < total) issue(jb + 1);
    if constexpr (GREG) {
#pragma unroll
      for (int it = 0; it < NI; ++it) {
        if (threadIdx.x + 256u * it >= items) break;
        const float g[2][2] = {{gc[it][0], gc[it][1]}, {gc[it][2], gc[it][3]}};
        block(ia[it], ib[it], g);
      }
    } else {
      for (uint32_t e = threadIdx.x; e < items; e += 256) {
        const uint32_t a = fdiv(e, dBW), b2 = e - a * (LGW / 2);
        float g[2][2];
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
          for (int cc = 0; cc < 2; ++cc)
            g[r][cc] = sg[(2 * a + r) * LGW + (cc % PG) * (LGW / PG) + (2 / PG) * b2 + cc / PG];
        block(a, b2, g);
      }
    }
  }
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int q = 0; q < T; ++q) {
    const float t = wave_reduce(acc[q]);
    if (lane == 0) red[wv][q] = t;
  }
  __syncthreads();
  if (threadIdx.x < T) {
    const int q = threadIdx.x;
    const double t = (double(red[0][q]) + double(red[1][q])) + (double(red[2][q]) + double(red[3][q]));
    part[(size_t(c) * npieces + piece) * T + q] = t;
  }
}

// Band-path geometry (0 rows: use the generic kernels).  Eligible shapes:
// K in {3, 5}, S in {1, 2}, p < K, the natural output size, operands below
// kOob floats, and windows that fit the LDS / register budget with bands of
// at least 2 rows (RB is even).
struct DwBand {
  uint32_t RB, R, LW, R2, LW2;  // dX: window R x LW; filter: x R x LW, dy R2 x LW2
  bool v4;                      // quad windows: LW, LW2 are the stored widths
};
static uint32_t round4(uint32_t v) { return (v + 3) & ~3u; }
static bool dw_band_ok(const DwGeom& g) {
  if (g.kH != g.kW || (g.kH != 3 && g.kH != 5) || (g.s != 1 && g.s != 2) || g.p >= g.kH)
    return false;
  if (g.H + 2 * g.p < g.kH || g.OH != (g.H + 2 * g.p - g.kH) / g.s + 1) return false;
  return uint64_t(g.B) * g.C * g.H * g.W < kOob && uint64_t(g.B) * g.C * g.OH * g.OW < kOob;
}
// The dX band kernels take kDwCW output columns per thread.
constexpr uint32_t kDwCW = 4;
static DwBand dw_band_input(const DwGeom& g) {
  DwBand b{0, 0, 0, 0, 0, false};
  if (!dw_band_ok(g)) return b;
  const uint32_t K = g.kH, BW = (g.W + kDwCW - 1) / kDwCW;
  const uint32_t WR = g.s == 1 ? K + 1 : ((1 + (g.p & 1)) / 2 + (K - (g.p & 1)) / 2 + 1);
  // Columns the last thread's window reaches (plus one).
  b.LW = g.s == 1 ? kDwCW * BW + K : (kDwCW / 2) * BW + WR;
  // Quad windows when dy rows are 4-aligned: the stored window starts at the
  // 4-aligned column left of the logical start cb.
  b.v4 = g.OW % 4 == 0;
  if (b.v4) {
    const int cb = g.s == 1 ? int(g.p) - int(K - 1) : int(g.p / 2) - int((K - (g.p & 1)) / 2);
    b.LW = round4(b.LW + uint32_t(cb & 3));
  }
  const uint32_t rows = kDwBand / b.LW;  // window rows that fit
  uint32_t RB = g.s == 1 ? (rows > K ? rows - K : 0) : (rows > WR ? 2 * (rows - WR) : 0);
  RB &= ~1u;
  if (RB < 2) return DwBand{0, 0, 0, 0, 0, false};
  RB = std::min(RB, (g.H + 1) & ~1u);
  b.RB = RB;
  b.R = g.s == 1 ? RB + K : RB / 2 + WR;
  return b;
}
static DwBand dw_band_fwd(const DwGeom& g) {
  DwBand b{0, 0, 0, 0, 0, false};
  if (!dw_band_ok(g)) return b;
  const uint32_t K = g.kH, S = g.s, BW = (g.OW + 1) / 2;
  b.LW = (2 * BW - 1) * S + K;
  // Quad windows when x rows are 4-aligned: the stored window starts at the
  // 4-aligned column left of -p.
  b.v4 = g.W % 4 == 0;
  if (b.v4) b.LW = round4(b.LW + uint32_t(-int(g.p) & 3));
  const uint32_t rows = kDwBand / b.LW;  // window rows that fit
  uint32_t RB = rows >= K ? ((rows - K) / S + 1) & ~1u : 0;
  if (RB < 2) return DwBand{0, 0, 0, 0, 0, false};
  RB = std::min(RB, (g.OH + 1) & ~1u);
  b.RB = RB;
  b.R = (RB - 1) * S + K;
  return b;
}
static DwBand dw_band_filter(const DwGeom& g) {
  DwBand b{0, 0, 0, 0, 0, false};
  if (!dw_band_ok(g)) return b;
  const uint32_t K = g.kH, S = g.s;
  b.LW2 = (g.OW + 1) & ~1u;
  b.LW = (b.LW2 - 1) * S + K;
  // Quad windows when x and dy rows are 4-aligned (LW2 = OW is then a
  // multiple of 4; the x window starts at the 4-aligned column left of -p).
  b.v4 = g.W % 4 == 0 && g.OW % 4 == 0;
  if (b.v4)
    b.LW = round4(b.LW + uint32_t(-int(g.p) & 3));
  else
    b.LW = S == 2 ? round4(b.LW) : b.LW;  // stride-2 phase-split rows need LW % 4 == 0
  if (b.LW2 * 2 > dw_gband(S) || uint64_t(b.LW) * (S + K) > kDwBand) return DwBand{0, 0, 0, 0, 0, false};
  const uint32_t byg = dw_gband(S) / b.LW2;
  const uint32_t byx = (kDwBand / b.LW - K) / S + 1;
  uint32_t RB = std::min(byg, byx) & ~1u;
  if (RB < 2) return DwBand{0, 0, 0, 0, 0, false};
  RB = std::min(RB, (g.OH + 1) & ~1u);
  b.RB = RB;
  b.R2 = RB;
  b.R = (RB - 1) * S + K;
  return b;
}

static bool dw_ok(const DwGeom& g, const char* what) {
  if (!g.B || !g.C || !g.H || !g.W || !g.kH || !g.kW || !g.s || !g.OH || !g.OW) return false;
  if (uint64_t(g.B) * g.C * std::max(uint64_t(g.H) * g.W, uint64_t(g.OH) * g.OW) >= (1ull << 31)) {
    set_error("%s: tensor too large", what);
    return false;
  }
  return true;
}
static bool sh_dw_fwd(const Dispatch& d) {
  DwGeom g = dw_geom(d);
  if (!dw_ok(g, "depthwise_conv_forward")) return true;
  uint32_t total = g.B * g.C * g.OH * g.OW;
  const Buf x = S(d, 0), f = S(d, 1), bias = S(d, 2), y = U(d, 0);
  const DwBand bb = dw_band_fwd(g);
  const uint32_t nx = g.B * g.C * g.H * g.W;
  if (bb.RB && covers(x, nx) && covers(f, uint64_t(g.C) * g.kH * g.kW) && covers(bias, g.C) &&
      covers(y, total)) {
    const uint32_t nb = cdiv(g.OH, bb.RB), nbands = g.B * g.C * nb;
    const uint32_t BW = (g.OW + 1) / 2;
    const FastDiv fLW = make_fastdiv(bb.v4 ? bb.LW / 4 : bb.LW), fNb = make_fastdiv(nb),
                  fBW = make_fastdiv(BW);
    // The batch-norm statistics of y ride along (a BN usually follows): a
    // side buffer of C * B * nb double pairs, owned by y once the launch is
    // made.
    const uint32_t pieces = g.B * nb;
    Buffer* side = nullptr;
    if (d.nU && uint64_t(g.C) * pieces * 4 < 0xFFFFFFFFull)
      side = static_cast<Buffer*>(create_buffer(nullptr, g.C * pieces * 4));
    double* stats = side ? reinterpret_cast<double*>(side->ptr) : nullptr;
    // One block per band, in band order (as the dX band kernel).
#define DCE_DWF_V(K, SS, V)                                                                      \
  {                                                                                             \
    const uint32_t blocks = nbands;                                                             \
    if (stats)                                                                                  \
      hipLaunchKernelGGL((k_dw_fwd_band<K, SS, V, true>), dim3(blocks), dim3(256), 0, stream(),  \
                         x.p, f.p, bias.p, y.p, g.C, g.H, g.W, g.OH, g.OW, g.p, bb.RB, nb,       \
                         nbands, bb.R, bb.LW, BW, nx, fLW, fNb, fBW, stats);                     \
    else                                                                                        \
      hipLaunchKernelGGL((k_dw_fwd_band<K, SS, V, false>), dim3(blocks), dim3(256), 0, stream(), \
                         x.p, f.p, bias.p, y.p, g.C, g.H, g.W, g.OH, g.OW, g.p, bb.RB, nb,       \
                         nbands, bb.R, bb.LW, BW, nx, fLW, fNb, fBW, nullptr);                   \
  }
#define DCE_DWF(K, SS)                                                                           \
  if (g.kH == K && g.s == SS) {                                                                 \
    if (bb.v4)                                                                                  \
      DCE_DWF_V(K, SS, true)                                                                    \
    else                                                                                        \
      DCE_DWF_V(K, SS, false)                                                                   \
  }
    DCE_DWF(3, 1) DCE_DWF(3, 2) DCE_DWF(5, 1) DCE_DWF(5, 2)
#undef DCE_DWF
#undef DCE_DWF_V
    if (!check_launch("depthwise_conv_forward")) {
      release_buffer(side);
      return false;
    }
    if (side) tag_bn_stats(d.uavs[0], side, g.B, g.C, g.OH * g.OW, pieces);  // no conv G
    return true;
  }
  hipLaunchKernelGGL(k_dw_fwd, dim3(cdiv(total, 256)), dim3(256), 0, stream(), S(d, 0), S(d, 1),
                     S(d, 2), U(d, 0), g, total);
  return check_launch("depthwise_conv_forward");
}
static bool sh_dw_bwd_input(const Dispatch& d) {
  DwGeom g = dw_geom(d);
  if (!dw_ok(g, "depthwise_conv_backward_input")) return true;
  uint32_t total = g.B * g.C * g.H * g.W;
  ProfScope prof("dw_bwd_input", 2.0 * g.kH * g.kW * double(g.B) * g.C * g.OH * g.OW,
                 4.0 * double(total) + 4.0 * double(g.B) * g.C * g.OH * g.OW);
  const Buf dy = S(d, 0), f = S(d, 1), dx = U(d, 0);
  const DwBand bb = dw_band_input(g);
  if (bb.RB && covers(dy, uint64_t(g.B) * g.C * g.OH * g.OW) &&
      covers(f, uint64_t(g.C) * g.kH * g.kW) && covers(dx, total)) {
    const uint32_t nb = cdiv(g.H, bb.RB), nbands = g.B * g.C * nb;
    const uint32_t BW = (g.W + kDwCW - 1) / kDwCW, ndy = g.B * g.C * g.OH * g.OW;
    const FastDiv fLW = make_fastdiv(bb.v4 ? bb.LW / 4 : bb.LW), fNb = make_fastdiv(nb),
                  fBW = make_fastdiv(BW);
    const uint32_t podd = g.p & 1;
    // One block per band, in band (= memory) order: the blocks that run at
    // the same time then write neighbouring rows of dx.  Measured against a
    // resident round of blocks walking the bands with a grid stride (which
    // overlaps each block's next window load with its compute): 64x144x56x56
    // s1 40.6 -> 38.1 us, 64x96x112x112 s2 81.4 -> 77.0 us.  On a plain
    // 1.2 GB fill the same contrast is 6.85 against 4.4-5.0 TB/s.
    // Passes over more than the MALL store dx with the nontemporal policy.
    const bool nt = stream_nt(4.0 * (double(total) + ndy)) &&
                    (reinterpret_cast<uintptr_t>(dx.p) & 15) == 0;
#define DCE_DWI_NT(K, SS, PO, V, NT)                                                             \
  hipLaunchKernelGGL((k_dw_bwd_input_band<K, SS, PO, V, kDwCW, NT>), dim3(nbands), dim3(256), 0, \
                     stream(), dy.p, f.p, dx.p, g.C, g.H, g.W, g.OH, g.OW, g.p, bb.RB, nb,       \
                     nbands, bb.R, bb.LW, BW, ndy, fLW, fNb, fBW);
#define DCE_DWI_V(K, SS, PO, V)                                                                   \
  {                                                                                              \
    if (nt)                                                                                      \
      DCE_DWI_NT(K, SS, PO, V, true)                                                             \
    else                                                                                         \
      DCE_DWI_NT(K, SS, PO, V, false)                                                            \
  }
#define DCE_DWI(K, SS, PO)                                                                        \
  if (g.kH == K && g.s == SS && (SS == 1 || podd == PO)) {                                       \
    if (bb.v4)                                                                                   \
      DCE_DWI_V(K, SS, PO, true)                                                                 \
    else                                                                                         \
      DCE_DWI_V(K, SS, PO, false)                                                                \
  }
    DCE_DWI(3, 1, 0) DCE_DWI(3, 2, 0) DCE_DWI(3, 2, 1)
    DCE_DWI(5, 1, 0) DCE_DWI(5, 2, 0) DCE_DWI(5, 2, 1)
#undef DCE_DWI
#undef DCE_DWI_V
#undef DCE_DWI_NT
    return check_launch("depthwise_conv_backward_input");
  }
  hipLaunchKernelGGL(k_dw_bwd_input, dim3(cdiv(total, 256)), dim3(256), 0, stream(), dy, f, dx, g,
                     total);
  return check_launch("depthwise_conv_backward_input");
}
static bool sh_dw_bwd_filter(const Dispatch& d) {
  DwGeom g = dw_geom(d);
  if (!dw_ok(g, "depthwise_conv_backward_filter")) return true;
  const uint32_t taps = g.kH * g.kW;
  if (taps > uint32_t(kDwMaxTaps)) {
    set_error("depthwise_conv_backward_filter: kernels above 5x5 are not supported");
    return false;
  }
  const uint32_t len = g.B * g.OH * g.OW;
  const Buf dy = S(d, 0), x = S(d, 1);
  const DwBand bb = dw_band_filter(g);
  if (bb.RB && covers(dy, uint64_t(len) * g.C) && covers(x, uint64_t(g.B) * g.C * g.H * g.W)) {
    // Pieces per channel: one resident round of blocks over all channels (the
    // runtime's occupancy; a partly filled second round would run at a
    // fraction of the machine), each piece an even share of the channel's
    // (image, band) units, at least about one image's worth.
    int occ = 1;
#define DCE_DWO(K, SS)                                                                      \
  if (g.kH == K && g.s == SS)                                                              \
    occ = bb.v4 ? blocks_per_cu(k_dw_bwd_filter_band<K, SS, true, false>, 256)             \
                : blocks_per_cu(k_dw_bwd_filter_band<K, SS, false, false>, 256);
    DCE_DWO(3, 1) DCE_DWO(3, 2) DCE_DWO(5, 1) DCE_DWO(5, 2)
#undef DCE_DWO
    const uint32_t want =
        std::max<uint32_t>(1, uint32_t(num_cus()) * uint32_t(occ) / std::max<uint32_t>(1, g.C));
    // Stride 2 takes one image per piece instead (64x96x112x112: 73.8 ->
    // 70.4 us; stride 1 measured slower that way, 45.7 -> 49.6 us).  The
    // grid runs channels fastest, so the blocks that run together read the
    // planes of one image.
    const uint32_t pieces = g.s == 2 ? g.B : std::min<uint32_t>(g.B, want);
    double* part = reinterpret_cast<double*>(workspace(size_t(g.C) * pieces * (taps + 1) * 2));
    if (!part) return false;
    const double bytes = 4.0 * double(len) * g.C + 4.0 * double(g.B) * g.C * g.H * g.W;
    ProfScope prof("dw_bwd_filter", 2.0 * taps * double(len) * g.C, bytes);
    const bool nt = stream_nt(bytes);
    const dim3 grid(g.C, pieces);
    const uint32_t nb = cdiv(g.OH, bb.RB);
    const FastDiv fLX = make_fastdiv(bb.v4 ? bb.LW / 4 : bb.LW),
                  fLG = make_fastdiv(bb.v4 ? bb.LW2 / 4 : bb.LW2), fNb = make_fastdiv(nb),
                  fBW = make_fastdiv(bb.LW2 / 2);
#define DCE_DWF_N(K, SS, V, N)                                                                   \
  hipLaunchKernelGGL((k_dw_bwd_filter_band<K, SS, V, N>), grid, dim3(256), 0, stream(), dy.p, x.p,\
                     part, g.B, g.C, g.H, g.W, g.OH, g.OW, g.p, bb.RB, nb, bb.R, bb.LW, bb.R2,    \
                     bb.LW2, fLX, fLG, fNb, fBW);
#define DCE_DWF_V(K, SS, V)                                                                      \
  {                                                                                              \
    if (nt && V)                                                                                 \
      DCE_DWF_N(K, SS, V, true)                                                                  \
    else                                                                                         \
      DCE_DWF_N(K, SS, V, false)                                                                 \
  }
#define DCE_DWF(K, SS)                                                                          \
  if (g.kH == K && g.s == SS) {                                                                \
    if (bb.v4)                                                                                 \
      DCE_DWF_V(K, SS, true)                                                                   \
    else                                                                                       \
      DCE_DWF_V(K, SS, false)                                                                  \
  }
    DCE_DWF(3, 1) DCE_DWF(3, 2) DCE_DWF(5, 1) DCE_DWF(5, 2)
#undef DCE_DWF
#undef DCE_DWF_V
#undef DCE_DWF_N
    hipLaunchKernelGGL(k_dw_bwd_filter_final, dim3(cdiv(g.C * (taps + 1), 4)), dim3(256), 0,
                       stream(), part, pieces, g.C, taps, U(d, 0), U(d, 1));
    return check_launch("depthwise_conv_backward_filter");
  }
  const uint32_t pieces = std::max<uint32_t>(1, std::min<uint32_t>(cdiv(len, 8192), 128));
  double* part = reinterpret_cast<double*>(workspace(size_t(g.C) * pieces * (taps + 1) * 2));
  if (!part) return false;
  ProfScope prof("dw_bwd_filter", 2.0 * taps * double(len) * g.C,
                 4.0 * double(len) * g.C + 4.0 * double(g.B) * g.C * g.H * g.W);
  hipLaunchKernelGGL(k_dw_bwd_filter_part, dim3(pieces, g.C), dim3(256), 0, stream(), S(d, 0),
                     S(d, 1), g, pieces, part);
  hipLaunchKernelGGL(k_dw_bwd_filter_final, dim3(cdiv(g.C * (taps + 1), 4)), dim3(256), 0,
                     stream(), part, pieces, g.C, taps, U(d, 0), U(d, 1));
  return check_launch("depthwise_conv_backward_filter");
}

// ===========================================================================
// im2col / col2im / conv reshapes (RunShader compatibility; the fused conv
// path never materialises these).
// ===========================================================================
struct ColGeom {
  uint32_t B, C, H, W, k, s, p, OH, OW;
};
static ColGeom col_geom(const Dispatch& d) {
  return ColGeom{CU(d, 0), CU(d, 1), CU(d, 2), CU(d, 3), CU(d, 4), CU(d, 5), CU(d, 6), CU(d, 7), CU(d, 8)};
}
__global__ void k_im2col(Buf x, Buf col, ColGeom g, uint32_t total) {
  const uint32_t i = gtid();
  if (i >= total) return;
  const uint32_t tc = g.B * g.OH * g.OW;
  const uint32_t row = i / tc, cl = i - row * tc;
  const uint32_t b = cl / (g.OH * g.OW), pix = cl - b * g.OH * g.OW, oh = pix / g.OW,
                 ow = pix - oh * g.OW;
  const uint32_t ic = row / (g.k * g.k), kk = row - ic * g.k * g.k, kh = kk / g.k, kw = kk - kh * g.k;
  const int ih = int(oh * g.s + kh) - int(g.p), iw = int(ow * g.s + kw) - int(g.p);
  float v = 0.f;
  if (ih >= 0 && ih < int(g.H) && iw >= 0 && iw < int(g.W))
    v = ld(x, ((b * g.C + ic) * g.H + uint32_t(ih)) * g.W + uint32_t(iw));
  st(col, i, v);
}
__global__ void k_col2im(Buf col, Buf dx, ColGeom g, uint32_t total) {
  const uint32_t i = gtid();
  if (i >= total) return;
  const uint32_t iw = i % g.W, t = i / g.W, ih = t % g.H, t2 = t / g.H, ic = t2 % g.C, b = t2 / g.C;
  const uint32_t tc = g.B * g.OH * g.OW;
  float s = 0.f;
  for (uint32_t kh = 0; kh < g.k; ++kh)
    for (uint32_t kw = 0; kw < g.k; ++kw) {
      const int ohs = int(ih) - int(kh) + int(g.p), ows = int(iw) - int(kw) + int(g.p);
      if (ohs % int(g.s) == 0 && ows % int(g.s) == 0) {
        const uint32_t oh = uint32_t(ohs / int(g.s)), ow = uint32_t(ows / int(g.s));
        if (oh < g.OH && ow < g.OW)
          s += ld(col, (ic * g.k * g.k + kh * g.k + kw) * tc + b * g.OH * g.OW + oh * g.OW + ow);
      }
    }
  st(dx, i, s);
}
static bool sh_im2col(const Dispatch& d) {
  ColGeom g = col_geom(d);
  uint64_t total = uint64_t(g.C) * g.k * g.k * g.B * g.OH * g.OW;
  if (!total || !g.s || total >= (1ull << 32)) return true;
  hipLaunchKernelGGL(k_im2col, dim3(cdiv(total, 256)), dim3(256), 0, stream(), S(d, 0), U(d, 0), g,
                     uint32_t(total));
  return check_launch("im2col");
}
static bool sh_col2im(const Dispatch& d) {
  ColGeom g = col_geom(d);
  uint64_t total = uint64_t(g.B) * g.C * g.H * g.W;
  if (!total || !g.s || total >= (1ull << 32)) return true;
  hipLaunchKernelGGL(k_col2im, dim3(cdiv(total, 256)), dim3(256), 0, stream(), S(d, 0), U(d, 0), g,
                     uint32_t(total));
  return check_launch("col2im");
}
// conv_reshape: y[b, oc, pix] = act(mm[oc, b*OHW + pix] + bias[oc])
__global__ void k_conv_reshape(Buf mm, Buf bias, Buf y, uint32_t B, uint32_t OC, uint32_t OHW,
                               uint32_t act) {
  const uint32_t i = gtid();
  if (i >= B * OC * OHW) return;
  const uint32_t pix = i % OHW, t = i / OHW, oc = t % OC, b = t / OC;
  float z = ld(mm, oc * B * OHW + b * OHW + pix) + ld(bias, oc);
  if (act == 1) z = fmaxf(0.f, z);
  else if (act == 2) z = tanhf(z);
  st(y, i, z);
}
static bool sh_conv_reshape(const Dispatch& d) {
  uint32_t B = CU(d, 0), OC = CU(d, 1), OHW = CU(d, 2) * CU(d, 3);
  uint64_t n = uint64_t(B) * OC * OHW;
  if (!n) return true;
  hipLaunchKernelGGL(k_conv_reshape, dim3(cdiv(n, 256)), dim3(256), 0, stream(), S(d, 0), S(d, 1),
                     U(d, 0), B, OC, OHW, CU(d, 4));
  return check_launch("conv_reshape");
}
// conv_grad_reshape(_relu): G[oc, b*OHW + pix] = dZ[b, oc, pix] (masked where y <= 0)
template <bool RELU>
__global__ void k_conv_grad_reshape(Buf dz, Buf y, Buf g, uint32_t B, uint32_t OC, uint32_t OHW) {
  const uint32_t i = gtid();
  if (i >= B * OC * OHW) return;
  const uint32_t pix = i % OHW, t = i / OHW, oc = t % OC, b = t / OC;
  float v = ld(dz, i);
  if (RELU && ld(y, i) <= 0.f) v = 0.f;
  st(g, oc * B * OHW + b * OHW + pix, v);
}
template <bool RELU>
static bool sh_conv_grad_reshape(const Dispatch& d) {
  uint32_t B = CU(d, 0), OC = CU(d, 4), OHW = CU(d, 7) * CU(d, 8);
  uint64_t n = uint64_t(B) * OC * OHW;
  if (!n) return true;
  hipLaunchKernelGGL(k_conv_grad_reshape<RELU>, dim3(cdiv(n, 256)), dim3(256), 0, stream(),
                     S(d, 0), RELU ? S(d, 1) : Buf{nullptr, 0}, U(d, 0), B, OC, OHW);
  return check_launch("conv_grad_reshape");
}

// ===========================================================================
// Flagged GEMM shaders (matmul_universal / heavy / dgpu / coarsened / reduce):
// C = op(A)·op(B), constants {M, K, N, flags}.  Routed to the MFMA GEMM when
// every buffer covers the shape; otherwise a bounds-checked reference loop.
// ===========================================================================
__global__ void k_gemm_checked(Buf A, Buf B, Buf C, uint32_t M, uint32_t K, uint32_t N,
                               uint32_t flags) {
  const uint32_t i = gtid();
  if (i >= M * N) return;
  const uint32_t m = i / N, n = i - m * N;
  float s = 0.f;
  for (uint32_t k = 0; k < K; ++k) {
    const float a = ld(A, (flags & 1) ? k * M + m : m * K + k);
    const float b = ld(B, (flags & 2) ? n * K + k : k * N + n);
    s += a * b;
  }
  st(C, i, s);
}
// ===========================================================================
// Direct valid convolutions (stride 1, no padding, square kernel ks):
// conv_forward_tiled, conv_backprop_filters_tiled, conv_backprop_input_fused.
// All three share the constants {batch, inC, inH, inW, outC, ks, outH, outW,
// act}.  When outH = inH - ks + 1, outW = inW - ks + 1 and every buffer holds
// its geometry they run on the implicit-GEMM core (conv_forward /
// conv_backward); otherwise on the checked kernels below, which follow the
// shaders' flat index arithmetic (32-bit, wrapping) with the D3D11 rule of
// reads past a buffer returning 0 and writes past it dropped.
// ===========================================================================
struct TiledGeom {
  uint32_t B, C, H, W, OC, k, OH, OW;
};
static TiledGeom tiled_geom(const Dispatch& d) {
  return TiledGeom{CU(d, 0), CU(d, 1), CU(d, 2), CU(d, 3), CU(d, 4), CU(d, 5), CU(d, 6), CU(d, 7)};
}
static bool tiled_valid(const TiledGeom& g) {
  return g.k && g.H >= g.k && g.W >= g.k && g.OH == g.H - g.k + 1 && g.OW == g.W - g.k + 1 &&
         g.B && g.C && g.OC;
}
static ConvGeom tiled_conv(const TiledGeom& g) {
  return ConvGeom{g.B, g.C, g.H, g.W, g.OC, g.k, 1, 0, g.OH, g.OW};
}
__device__ __forceinline__ float tiled_act(float z, uint32_t act) {
  if (act == 1) return fmaxf(0.f, z);
  if (act == 2) return tanhf(z);
  return z;
}
// nn_conv_forward_tiled.hlsl:22-71: out[b, oc, pix] = act(Σ_k F[oc, k]·X(k, b, pix) + bias[oc]).
__global__ void k_conv_tiled_fwd_checked(Buf x, Buf f, Buf bias, Buf out, TiledGeom g,
                                         uint32_t act) {
  const uint32_t N = g.B * g.OH * g.OW, K = g.C * g.k * g.k;
  const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= uint64_t(N) * g.OC) return;
  const uint32_t row = uint32_t(i / N), col = uint32_t(i - uint64_t(row) * N);
  const uint32_t b = col / (g.OH * g.OW), pix = col % (g.OH * g.OW), oh = pix / g.OW,
                 ow = pix % g.OW;
  float acc = 0.f;
  for (uint32_t t = 0; t < K; ++t) {
    const uint32_t ic = t / (g.k * g.k), kk = t % (g.k * g.k), kh = kk / g.k, kw = kk % g.k;
    acc += ld(f, row * K + t) *
           ld(x, b * (g.C * g.H * g.W) + ic * (g.H * g.W) + (oh + kh) * g.W + (ow + kw));
  }
  st(out, b * (g.OC * g.OH * g.OW) + row * (g.OH * g.OW) + pix, tiled_act(acc + ld(bias, row), act));
}
// nn_conv_backprop_filters_tiled.hlsl:21-74: dF[oc, t] = Σ_{b, pix} dZ[b, oc, pix]·X(t, b, pix).
__global__ void k_conv_tiled_dw_checked(Buf dz, Buf x, Buf df, TiledGeom g) {
  const uint32_t N = g.B * g.OH * g.OW, tr = g.C * g.k * g.k;
  const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= uint64_t(tr) * g.OC) return;
  const uint32_t row = uint32_t(i / tr), col = uint32_t(i - uint64_t(row) * tr);
  const uint32_t ic = col / (g.k * g.k), kk = col % (g.k * g.k), kh = kk / g.k, kw = kk % g.k;
  float acc = 0.f;
  for (uint32_t t = 0; t < N; ++t) {
    const uint32_t b = t / (g.OH * g.OW), pix = t % (g.OH * g.OW), oh = pix / g.OW,
                   ow = pix % g.OW;
    acc += ld(dz, b * (g.OC * g.OH * g.OW) + row * (g.OH * g.OW) + pix) *
           ld(x, b * (g.C * g.H * g.W) + ic * (g.H * g.W) + (oh + kh) * g.W + (ow + kw));
  }
  st(df, row * tr + col, acc);
}
// The derivative factor of nn_conv_backprop_input_fused.hlsl:45-49, from the
// previous layer's activation output a: ReLU 1 or 0, tanh 1 - a², else 1.
struct OpPrevActGrad {
  uint32_t act;
  __device__ float operator()(float g, float a) const {
    float dA = 1.0f;
    if (act == 1) dA = a > 0.f ? 1.0f : 0.0f;
    else if (act == 2) dA = 1.0f - a * a;
    return g * dA;
  }
};
// nn_conv_backprop_input_fused.hlsl:19-50, one thread per input element.
__global__ void k_conv_tiled_dx_checked(Buf dz, Buf f, Buf aprev, Buf dx, TiledGeom g,
                                        uint32_t act) {
  const uint32_t total = g.B * g.C * g.H * g.W;
  const uint32_t i = gtid();
  if (i >= total) return;
  const uint32_t iw = i % g.W, ih = (i / g.W) % g.H, ic = (i / (g.W * g.H)) % g.C,
                 b = i / (g.C * g.H * g.W);
  float acc = 0.f;
  for (uint32_t oc = 0; oc < g.OC; ++oc)
    for (uint32_t kh = 0; kh < g.k; ++kh) {
      const int oh = int(ih) - int(kh);
      if (oh < 0 || oh >= int(g.OH)) continue;
      for (uint32_t kw = 0; kw < g.k; ++kw) {
        const int ow = int(iw) - int(kw);
        if (ow < 0 || ow >= int(g.OW)) continue;
        acc += ld(dz, b * (g.OC * g.OH * g.OW) + oc * (g.OH * g.OW) + uint32_t(oh) * g.OW +
                          uint32_t(ow)) *
               ld(f, oc * (g.C * g.k * g.k) + ic * (g.k * g.k) + kh * g.k + kw);
      }
    }
  st(dx, i, OpPrevActGrad{act}(acc, ld(aprev, i)));
}

static bool sh_conv_forward_tiled(const Dispatch& d) {
  const TiledGeom g = tiled_geom(d);
  const uint32_t act = CU(d, 8);
  const uint64_t n = uint64_t(g.B) * g.OH * g.OW * g.OC;
  if (!n) return true;
  Buf x = S(d, 0), f = S(d, 1), bias = S(d, 2), y = U(d, 0);
  if (tiled_valid(g) && covers(x, uint64_t(g.B) * g.C * g.H * g.W) &&
      covers(f, uint64_t(g.OC) * g.C * g.k * g.k) && covers(bias, g.OC) && covers(y, n))
    return conv_forward(x.p, nullptr, f.p, bias.p, y.p, tiled_conv(g), act <= 2 ? act : 0);
  hipLaunchKernelGGL(k_conv_tiled_fwd_checked, dim3(uint32_t(cdiv(n, 256))), dim3(256), 0,
                     stream(), x, f, bias, y, g, act);
  return check_launch("conv_forward_tiled");
}
// t0 = dZ, t1 = A_prev; u0 = dF, u1 = dB (bound by the reference's dispatch
// but never written by its shader, so it is left untouched here too).
static bool sh_conv_backprop_filters_tiled(const Dispatch& d) {
  const TiledGeom g = tiled_geom(d);
  const uint64_t n = uint64_t(g.OC) * g.C * g.k * g.k;
  if (!n) return true;
  Buf dz = S(d, 0), x = S(d, 1), df = U(d, 0);
  if (tiled_valid(g) && covers(dz, uint64_t(g.B) * g.OC * g.OH * g.OW) &&
      covers(x, uint64_t(g.B) * g.C * g.H * g.W) && covers(df, n))
    return conv_backward(dz.p, nullptr, x.p, nullptr, nullptr, df.p, nullptr, nullptr,
                         tiled_conv(g));
  hipLaunchKernelGGL(k_conv_tiled_dw_checked, dim3(uint32_t(cdiv(n, 256))), dim3(256), 0,
                     stream(), dz, x, df, g);
  return check_launch("conv_backprop_filters_tiled");
}
// t0 = dZ, t1 = filters, t2 = A_prev (the previous layer's activation
// output); u0 = dInput.  The derivative of the previous activation (act
// word: 1 ReLU, 2 tanh) multiplies the transposed convolution.
static bool sh_conv_backprop_input_fused(const Dispatch& d) {
  const TiledGeom g = tiled_geom(d);
  const uint32_t act = CU(d, 8);
  const uint64_t n = uint64_t(g.B) * g.C * g.H * g.W;
  if (!n || n >= (1ull << 32)) return n == 0;
  Buf dz = S(d, 0), f = S(d, 1), a = S(d, 2), dx = U(d, 0);
  if (tiled_valid(g) && covers(dz, uint64_t(g.B) * g.OC * g.OH * g.OW) &&
      covers(f, uint64_t(g.OC) * g.C * g.k * g.k) && covers(a, n) && covers(dx, n)) {
    if (!conv_backward(dz.p, nullptr, a.p, nullptr, f.p, nullptr, nullptr, dx.p, tiled_conv(g)))
      return false;
    if (act != 1 && act != 2) return true;
    return run_ew("conv_prev_act_grad", OpPrevActGrad{act}, dx, dx, a, uint32_t(n), false);
  }
  hipLaunchKernelGGL(k_conv_tiled_dx_checked, dim3(uint32_t(cdiv(n, 256))), dim3(256), 0,
                     stream(), dz, f, a, dx, g, act);
  return check_launch("conv_backprop_input_fused");
}

static bool sh_matmul(const Dispatch& d) {
  uint32_t M = CU(d, 0), K = CU(d, 1), N = CU(d, 2), flags = CU(d, 3) & 3u;
  uint64_t mn = uint64_t(M) * N;
  if (!mn) return true;
  Buf A = S(d, 0), B = S(d, 1), C = U(d, 0);
  if (covers(A, uint64_t(M) * K) && covers(B, uint64_t(K) * N) && covers(C, mn))
    return gemm(A.p, B.p, C.p, M, K, N, flags);
  if (mn >= (1ull << 32)) return false;
  hipLaunchKernelGGL(k_gemm_checked, dim3(cdiv(mn, 256)), dim3(256), 0, stream(), A, B, C, M, K, N,
                     flags);
  return check_launch("matmul");
}

// ===========================================================================
// Optimiser shaders (single tensor, RunShader form)
// ===========================================================================
__global__ void k_sgd(Buf w, Buf g, uint32_t n, float lr, float clip) {
  const uint32_t i = gtid();
  if (i >= n) return;
  float gv = ld(g, i);
  if (gv > clip) gv = clip;
  if (gv < -clip) gv = -clip;
  st(w, i, ld(w, i) - lr * gv);
}
static bool sh_sgd(const Dispatch& d) {  // cb {count, lr, clip, pad}; u0 = weight, t0 = grad
  uint32_t n = CU(d, 0);
  if (!n) return true;
  hipLaunchKernelGGL(k_sgd, dim3(cdiv(n, 256)), dim3(256), 0, stream(), U(d, 0), S(d, 0), n,
                     CF(d, 1), CF(d, 2));
  return check_launch("sgd");
}
__global__ void k_sgd_clipped(Buf w, Buf g, Buf ns, uint32_t n, float lr) {
  const uint32_t i = gtid();
  if (i < n) st(w, i, ld(w, i) - lr * ld(g, i) * ld(ns, 1));
}
static bool sh_sgd_clipped(const Dispatch& d) {
  uint32_t n = CU(d, 0);
  if (!n) return true;
  hipLaunchKernelGGL(k_sgd_clipped, dim3(cdiv(n, 256)), dim3(256), 0, stream(), U(d, 0), S(d, 0),
                     S(d, 1), n, CF(d, 1));
  return check_launch("sgd_clipped");
}
// One partial Σg² per 256-element group at globalOffset + group.
__global__ void k_grad_sq_reduce(Buf g, Buf part, uint32_t n, uint32_t off) {
  __shared__ double sh[4];
  const uint32_t i = gtid();
  const float v = i < n ? ld(g, i) : 0.f;
  const double s = block_sum256(double(v * v), sh);
  if (threadIdx.x == 0) st(part, off + blockIdx.x, float(s));
}
static bool sh_grad_sq_reduce(const Dispatch& d) {
  uint32_t n = CU(d, 0);
  if (!n) return true;
  hipLaunchKernelGGL(k_grad_sq_reduce, dim3(cdiv(n, 256)), dim3(256), 0, stream(), S(d, 0), U(d, 0),
                     n, CU(d, 1));
  return check_launch("grad_sq_reduce");
}
__global__ void k_grad_norm_final(Buf part, Buf ns, uint32_t total, float maxNorm) {
  __shared__ double sh[4];
  double s = 0;
  for (uint32_t i = threadIdx.x; i < total; i += 256) s += ld(part, i);
  s = block_sum256(s, sh);
  if (threadIdx.x == 0) {
    const float norm = sqrtf(float(s));
    st(ns, 0, norm);
    st(ns, 1, (norm > maxNorm) ? (maxNorm / (norm + 1e-6f)) : 1.0f);
  }
}
static bool sh_grad_norm_final(const Dispatch& d) {
  hipLaunchKernelGGL(k_grad_norm_final, dim3(1), dim3(256), 0, stream(), S(d, 0), U(d, 0),
                     CU(d, 0), CF(d, 1));
  return check_launch("grad_norm_final");
}
__global__ void k_adam(Buf w, Buf m, Buf v, Buf g, uint32_t n, float step, float b1, float b2,
                       float eps, float wd, float clip) {
  const uint32_t i = gtid();
  if (i >= n) return;
  float gv = ld(g, i);
  if (gv > clip) gv = clip;
  if (gv < -clip) gv = -clip;
  const float cw = ld(w, i);
  const float mt = b1 * ld(m, i) + (1.0f - b1) * gv;
  const float vt = b2 * ld(v, i) + (1.0f - b2) * gv * gv;
  st(m, i, mt);
  st(v, i, vt);
  st(w, i, cw - wd * cw - step * mt / (sqrtf(vt) + eps));
}
static bool sh_adam(const Dispatch& d) {  // u0 weight, u1 m, u2 v, t0 grad
  uint32_t n = CU(d, 0);
  if (!n) return true;
  hipLaunchKernelGGL(k_adam, dim3(cdiv(n, 256)), dim3(256), 0, stream(), U(d, 0), U(d, 1), U(d, 2),
                     S(d, 0), n, CF(d, 1), CF(d, 2), CF(d, 3), CF(d, 4), CF(d, 5), CF(d, 6));
  return check_launch("adam");
}
// rms: out[0] = sqrt(Σ A² / count) (nn_rms.hlsl)
__global__ void k_rms(Buf A, Buf out, uint32_t n) {
  __shared__ double sh[4];
  double s = 0;
  for (uint32_t i = threadIdx.x; i < n; i += 256) {
    const float v = ld(A, i);
    s += double(v * v);
  }
  s = block_sum256(s, sh);
  if (threadIdx.x == 0) st(out, 0, sqrtf(float(s) / float(n)));
}
static bool sh_rms(const Dispatch& d) {
  uint32_t n = CU(d, 0);
  if (!n) return true;
  hipLaunchKernelGGL(k_rms, dim3(1), dim3(256), 0, stream(), S(d, 0), U(d, 0), n);
  return check_launch("rms");
}

// ===========================================================================
// Registry (names of nn_engine.py:147-173 that have kernel sources)
// ===========================================================================
static const ShaderEntry kShaders[] = {
    {"matmul_universal", sh_matmul},
    {"matmul_coarsened", sh_matmul},
    {"matmul_heavy", sh_matmul},
    {"matmul_dgpu", sh_matmul},
    {"matmul_reduce", sh_matmul},
    {"add_bias", sh_add_bias_t<false>},
    {"bias_relu", sh_add_bias_t<true>},
    {"relu", sh_relu},
    {"relu_grad", sh_relu_grad},
    {"relu6", sh_relu6},
    {"relu6_grad", sh_relu6_grad},
    {"sigmoid", sh_sigmoid},
    {"sigmoid_grad", sh_sigmoid_grad},
    {"leaky_relu", sh_leaky},
    {"leaky_relu_grad", sh_leaky_grad},
    {"add", sh_add},
    {"scale_add", sh_scale_add},
    {"rms", sh_rms},
    {"grad_accum", sh_grad_accum},
    {"bias_grad", sh_bias_grad},
    {"softmax", sh_softmax},
    {"loss", sh_loss},
    {"softmax_ce_grad", sh_softmax_ce_grad},
    {"argmax_correct", sh_argmax_correct},
    {"accumulate_scalar", sh_accumulate_scalar},
    {"dice_loss", sh_dice_loss},
    {"dice_loss_sums", sh_dice_sums},
    {"dice_loss_grad", sh_dice_grad},
    {"batchnorm_mean_var", sh_bn_mean_var},
    {"batchnorm_forward", sh_bn_forward},
    {"batchnorm_backward_reduce", sh_bn_backward_reduce},
    {"batchnorm_backward_dx", sh_bn_backward_dx},
    {"maxpool_forward", sh_maxpool_forward},
    {"maxpool_backward", sh_maxpool_backward},
    {"global_avg_pool", sh_gap},
    {"global_avg_pool_backward", sh_gap_bwd},
    {"upsample", sh_upsample},
    {"upsample_backward", sh_upsample_bwd},
    {"concat_insert", sh_chan_copy<0>},
    {"slice", sh_chan_copy<1>},
    {"depthwise_conv_forward", sh_dw_fwd},
    {"depthwise_conv_backward_input", sh_dw_bwd_input},
    {"depthwise_conv_backward_filter", sh_dw_bwd_filter},
    {"im2col", sh_im2col},
    {"col2im", sh_col2im},
    {"conv_forward_tiled", sh_conv_forward_tiled},
    {"conv_backprop_filters_tiled", sh_conv_backprop_filters_tiled},
    {"conv_backprop_input_fused", sh_conv_backprop_input_fused},
    {"conv_reshape", sh_conv_reshape},
    {"conv_grad_reshape", sh_conv_grad_reshape<false>},
    {"conv_grad_reshape_relu", sh_conv_grad_reshape<true>},
    {"sgd", sh_sgd},
    {"sgd_clipped", sh_sgd_clipped},
    {"grad_sq_reduce", sh_grad_sq_reduce},
    {"grad_norm_final", sh_grad_norm_final},
    {"adam", sh_adam},
};

const ShaderEntry* find_shader(const char* name) {
  for (const ShaderEntry& e : kShaders)
    if (strcmp(e.name, name) == 0) return &e;
  return nullptr;
}

// A pointer is a registry entry only if it is the address of one element of
// the table; nothing behind it is read before this holds.
const ShaderEntry* shader_entry(const void* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p), lo = reinterpret_cast<uintptr_t>(kShaders);
  const size_t n = sizeof(kShaders) / sizeof(kShaders[0]);
  if (a < lo || a >= lo + n * sizeof(ShaderEntry) || (a - lo) % sizeof(ShaderEntry) != 0)
    return nullptr;
  return &kShaders[(a - lo) / sizeof(ShaderEntry)];
}

}  // namespace dce
