// fp32 implicit GEMM on CDNA4 matrix cores (v_mfma_f32_16x16x4_f32) for the
// convolution forward, filter gradient (dW), input gradient (dX) and the
// flagged dense GEMM of MatMulAlloc.
//
//   C[m, n] = sum_k A[m, k] * B[n, k]
//
// Workgroup: 256 threads = 4 wave64 in a 2x2 arrangement owning an MT x NT
// output tile (MT, NT in {64, 128}); each wave an (MT/2) x (NT/2) block of
// 16x16 accumulators.  K advances in tiles of KT (16 or 32) through a double
// buffered LDS stage with one barrier per tile; the next tile's global loads
// are in flight while the current one is multiplied.
//
// Every global load is a (predicated) 16-byte load of four consecutive
// elements ("quad").  An operand is staged in LDS in one of two layouts:
//   ROWK  [row][k], quads along k  (row stride KT + 4)   -> ds_read_b128
//   KROW  [k][row], quads along rows (k stride R + 4)    -> 4 x ds_read_b32
// Both feed the MFMA with the same k order: in MFMA s of a 16-wide k slice,
// lane l (r = l % 16, g = l / 16) supplies A[r][4g + s] and B[4g + s][r], so
// the four MFMAs together cover k 0..15 (the matrix unit sums over g).  The
// +4 paddings make both the quad stores and the fragment reads bank-conflict
// free for 8 (b128) or 32 (b32) consecutive lanes.
//
// Convolutions work on channel-innermost ("NHWC", channels padded to a
// multiple of 4) copies of their activations so that a quad is four
// consecutive channels of one pixel:
//   forward  A = filters [oc][(kh,kw,c)]      ROWK   B = x patches, rows = output pixels   ROWK
//   dX       A = filters [c][(kh,kw,oc)]      ROWK   B = G patches, rows = input pixels    ROWK
//   dW       A = G rows oc, k = pixels        KROW   B = x taps, rows (kh,kw,c), k = pixels KROW
// where G = dy masked by the ReLU output (y <= 0 -> 0), produced once per
// backward by a transpose pass that also reduces the bias gradient.  No
// im2col / col2im buffer exists; the NHWC copy of x is what ConvForwardFused
// hands back as its "im2col" handle.
// Split-K (blockIdx.z) writes partial tiles that a second pass sums in a
// fixed order; nothing uses atomics, so results are deterministic.
#include "dce_internal.h"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace dce {

typedef float f4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
static inline uint32_t cdiv(uint64_t a, uint64_t b) { return uint32_t((a + b - 1) / b); }

// ---------------------------------------------------------------------------
// LDS stage geometry of one operand.
// ---------------------------------------------------------------------------
template <int R, int KT, bool KROW>
struct Stage {
  static constexpr int LD = KROW ? (R + 4) : (KT + 4);
  static constexpr int SIZE = KROW ? KT * LD : R * LD;
  static constexpr int KQ = KT / 4;
  static constexpr int RQ = R / 4;
  static_assert((R * KT / 4) % kThreads == 0, "tile must split evenly over the workgroup");
  static constexpr int Q = R * KT / 4 / kThreads;
  // Quad i of thread t.  ROWK: consecutive lanes take consecutive k-quads of
  // one row; KROW: consecutive lanes take consecutive row-quads of one k.
  __device__ static __forceinline__ int qrow(int t, int i) {
    const int q = t + kThreads * i;
    return KROW ? 4 * (q % RQ) : q / KQ;
  }
  __device__ static __forceinline__ int qk(int t, int i) {
    const int q = t + kThreads * i;
    return KROW ? q / RQ : 4 * (q % KQ);
  }
  __device__ static __forceinline__ int lds_off(int t, int i) {
    return KROW ? qk(t, i) * LD + qrow(t, i) : qrow(t, i) * LD + qk(t, i);
  }
  // MFMA operand of 16 rows starting at rb, k slice kb: components s = 0..3.
  __device__ static __forceinline__ f4 frag(const float* S, int rb, int r, int g, int kb) {
    if (!KROW) return *reinterpret_cast<const f4*>(S + (rb + r) * LD + kb + 4 * g);
    f4 v;
#pragma unroll
    for (int s = 0; s < 4; ++s) v[s] = S[(kb + 4 * g + s) * LD + rb + r];
    return v;
  }
};

template <class St>
struct LoaderBase {
  static constexpr int Q = St::Q;
  int lds[Q];
  __device__ __forceinline__ void base_init(int tid) {
#pragma unroll
    for (int i = 0; i < Q; ++i) lds[i] = St::lds_off(tid, i);
  }
  __device__ __forceinline__ void store(float* S, const f4 (&r)[Q]) const {
#pragma unroll
    for (int i = 0; i < Q; ++i) *reinterpret_cast<f4*>(S + lds[i]) = r[i];
  }
};

__device__ __forceinline__ f4 zero4() { return f4{0.f, 0.f, 0.f, 0.f}; }
__device__ __forceinline__ f4 ld4(const float* p) { return *reinterpret_cast<const f4*>(p); }

// ---------------------------------------------------------------------------
// Dense operands.
// ---------------------------------------------------------------------------
// [rows][kdim] row-major (ROWK).  vec: ld % 4 == 0, kdim % 4 == 0, aligned.
template <int R, int KT>
struct LdDenseRK : LoaderBase<Stage<R, KT, false>> {
  using St = Stage<R, KT, false>;
  static constexpr bool KROW = false;
  using LoaderBase<St>::Q;
  struct Params {
    const float* p;
    uint32_t ld, rows, kdim, vec;
  };
  const float* p;
  uint32_t ld, kdim;
  bool vec;
  uint32_t row[Q], kq[Q];
  bool rok[Q];
  __device__ __forceinline__ void init(const Params& P, uint32_t row0, int tid) {
    this->base_init(tid);
    p = P.p;
    ld = P.ld;
    kdim = P.kdim;
    vec = P.vec != 0;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      row[i] = row0 + St::qrow(tid, i);
      kq[i] = St::qk(tid, i);
      rok[i] = row[i] < P.rows;
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t k0 = kt * KT + kq[i];
      if (vec) {
        r[i] = (rok[i] && k0 < kdim) ? ld4(p + row[i] * ld + k0) : zero4();
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          r[i][e] = (rok[i] && k0 + e < kdim) ? p[row[i] * ld + k0 + e] : 0.f;
      }
    }
  }
};

// [kdim][rows] k-major (KROW).  vec: rows % 4 == 0, ld % 4 == 0, aligned.
template <int R, int KT>
struct LdDenseKR : LoaderBase<Stage<R, KT, true>> {
  using St = Stage<R, KT, true>;
  static constexpr bool KROW = true;
  using LoaderBase<St>::Q;
  struct Params {
    const float* p;
    uint32_t ld, rows, kdim, vec;
  };
  const float* p;
  uint32_t ld, kdim, rows;
  bool vec;
  uint32_t row[Q], kk[Q];
  __device__ __forceinline__ void init(const Params& P, uint32_t row0, int tid) {
    this->base_init(tid);
    p = P.p;
    ld = P.ld;
    kdim = P.kdim;
    rows = P.rows;
    vec = P.vec != 0;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      row[i] = row0 + St::qrow(tid, i);
      kk[i] = St::qk(tid, i);
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t k = kt * KT + kk[i];
      if (vec) {
        r[i] = (k < kdim && row[i] < rows) ? ld4(p + k * ld + row[i]) : zero4();
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          r[i][e] = (k < kdim && row[i] + e < rows) ? p[k * ld + row[i] + e] : 0.f;
      }
    }
  }
};

// ---------------------------------------------------------------------------
// Pixel-row gather over an NHWC source (ROWK): rows = pixels of a grid
// (b, a, c), k = (kh, kw, ch) with ch fastest (ch padded to Cp % 4 == 0).
//   FWD: source = x, rows = output pixels, tap reads x[b, a*s + kh - p, c*s + kw - p].
//   !FWD (dX): source = G, rows = input pixels, tap reads G[b, oh, ow] with
//        oh*s == a + p - kh exactly (S1: s == 1, no divisibility test).
// ---------------------------------------------------------------------------
template <int R, int KT, bool FWD, bool S1>
struct LdPixRK : LoaderBase<Stage<R, KT, false>> {
  using St = Stage<R, KT, false>;
  static constexpr bool KROW = false;
  using LoaderBase<St>::Q;
  struct Params {
    const float* src;
    uint32_t srcH, srcW, Cp, k, s, p;
    uint32_t gridW, gridHW, N, kdim;
    FastDiv dGridHW, dGridW, dCp, dK;
  };
  const float* src;
  uint32_t srcH, srcW, Cp, k, s, kdim;
  FastDiv dCp, dK;
  uint32_t pbase[Q], kq[Q];
  int r0[Q], c0[Q];
  bool rok[Q];
  __device__ __forceinline__ void init(const Params& P, uint32_t row0, int tid) {
    this->base_init(tid);
    src = P.src;
    srcH = P.srcH;
    srcW = P.srcW;
    Cp = P.Cp;
    k = P.k;
    s = P.s;
    kdim = P.kdim;
    dCp = P.dCp;
    dK = P.dK;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t n = row0 + St::qrow(tid, i);
      kq[i] = St::qk(tid, i);
      rok[i] = n < P.N;
      const uint32_t b = fdiv(n, P.dGridHW);
      const uint32_t rem = n - b * P.gridHW;
      const uint32_t a = fdiv(rem, P.dGridW);
      const uint32_t c = rem - a * P.gridW;
      pbase[i] = b * P.srcH * P.srcW;
      if (FWD) {
        r0[i] = int(a * P.s) - int(P.p);
        c0[i] = int(c * P.s) - int(P.p);
      } else {
        r0[i] = int(a + P.p);
        c0[i] = int(c + P.p);
      }
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t kk0 = kt * KT + kq[i];
      const uint32_t khw = fdiv(kk0, dCp);
      const uint32_t ch = kk0 - khw * Cp;
      const uint32_t kh = fdiv(khw, dK);
      const uint32_t kw = khw - kh * k;
      int h, w;
      bool ok = rok[i] && kk0 < kdim;
      if (FWD) {
        h = r0[i] + int(kh);
        w = c0[i] + int(kw);
      } else if (S1) {
        h = r0[i] - int(kh);
        w = c0[i] - int(kw);
      } else {
        const int hs = r0[i] - int(kh), ws = c0[i] - int(kw);
        ok = ok && hs >= 0 && ws >= 0;
        h = int(uint32_t(hs) / s);
        w = int(uint32_t(ws) / s);
        ok = ok && uint32_t(h) * s == uint32_t(hs) && uint32_t(w) * s == uint32_t(ws);
      }
      ok = ok && uint32_t(h) < srcH && uint32_t(w) < srcW;
      r[i] = ok ? ld4(src + (pbase[i] + uint32_t(h) * srcW + uint32_t(w)) * Cp + ch) : zero4();
    }
  }
};

// ---------------------------------------------------------------------------
// dW operands (KROW, k = flat output pixel over the batch).
// ---------------------------------------------------------------------------
// A: G rows oc, element (oc, pix) = G_nhwc[pix*OCp + oc].
template <int R, int KT>
struct LdGradKR : LoaderBase<Stage<R, KT, true>> {
  using St = Stage<R, KT, true>;
  static constexpr bool KROW = true;
  using LoaderBase<St>::Q;
  struct Params {
    const float* g;
    uint32_t OCp, npix;
  };
  const float* g;
  uint32_t OCp, npix;
  uint32_t oc[Q], kk[Q];
  __device__ __forceinline__ void init(const Params& P, uint32_t row0, int tid) {
    this->base_init(tid);
    g = P.g;
    OCp = P.OCp;
    npix = P.npix;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      oc[i] = row0 + St::qrow(tid, i);
      kk[i] = St::qk(tid, i);
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t pix = kt * KT + kk[i];
      r[i] = (oc[i] < OCp && pix < npix) ? ld4(g + pix * OCp + oc[i]) : zero4();
    }
  }
};

// B: x taps, rows n = (kh, kw, c) (c fastest, Cp), element (n, pix) =
// x_nhwc[b, oh*s + kh - p, ow*s + kw - p, c] or 0 outside the image.
template <int R, int KT>
struct LdXTapKR : LoaderBase<Stage<R, KT, true>> {
  using St = Stage<R, KT, true>;
  static constexpr bool KROW = true;
  using LoaderBase<St>::Q;
  struct Params {
    const float* x;
    uint32_t H, W, Cp, k, s, p, OW, OHW, npix, N;
    FastDiv dOHW, dOW, dCp, dK;
  };
  const float* x;
  uint32_t H, W, Cp, s, OW, OHW, npix;
  FastDiv dOHW, dOW;
  uint32_t off[Q], kk[Q];
  int kh[Q], kw[Q];
  bool rok[Q];
  __device__ __forceinline__ void init(const Params& P, uint32_t row0, int tid) {
    this->base_init(tid);
    x = P.x;
    H = P.H;
    W = P.W;
    Cp = P.Cp;
    s = P.s;
    OW = P.OW;
    OHW = P.OHW;
    npix = P.npix;
    dOHW = P.dOHW;
    dOW = P.dOW;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t n = row0 + St::qrow(tid, i);
      kk[i] = St::qk(tid, i);
      rok[i] = n < P.N;
      const uint32_t khw = fdiv(n, P.dCp);
      off[i] = n - khw * P.Cp;
      const uint32_t a = fdiv(khw, P.dK);
      kh[i] = int(a) - int(P.p);
      kw[i] = int(khw - a * P.k) - int(P.p);
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t pix = kt * KT + kk[i];
      const uint32_t b = fdiv(pix, dOHW);
      const uint32_t rem = pix - b * OHW;
      const uint32_t oh = fdiv(rem, dOW);
      const uint32_t ow = rem - oh * OW;
      const int ih = int(oh * s) + kh[i];
      const int iw = int(ow * s) + kw[i];
      const bool ok = rok[i] && pix < npix && uint32_t(ih) < H && uint32_t(iw) < W;
      r[i] = ok ? ld4(x + ((b * H + uint32_t(ih)) * W + uint32_t(iw)) * Cp + off[i]) : zero4();
    }
  }
};

// ---------------------------------------------------------------------------
// Epilogues.  Lane l of wave (wm, wn) holds, for MFMA block (i, j) and
// register v, C[m0 + wm*MT/2 + 16i + 4(l/16) + v][n0 + wn*NT/2 + 16j + l%16].
// ---------------------------------------------------------------------------
struct EpiRowMajor {
  struct Params {
    float* c;
    uint32_t M, N, ldc, splitStride;
  };
  template <int MT, int NT, int FM, int FN>
  __device__ static __forceinline__ void store(const Params& p, const f4 (&acc)[FM][FN],
                                               uint32_t m0, uint32_t n0, uint32_t z, int wm,
                                               int wn, int lane) {
    float* c = p.c + size_t(z) * p.splitStride;
    const int r = lane & 15, g = lane >> 4;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const uint32_t n = n0 + wn * (NT / 2) + j * 16 + r;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const uint32_t m = m0 + wm * (MT / 2) + i * 16 + 4 * g + v;
          if (m < p.M && n < p.N) c[m * p.ldc + n] = acc[i][j][v];
        }
      }
    }
  }
};

// NCHW output: out[b][m][pix] for n = b*HW + pix; optional bias + activation
// (0 identity, 1 ReLU, 2 tanh), as nn_conv_reshape.hlsl:23-26.
struct EpiNCHW {
  struct Params {
    float* out;
    const float* bias;
    uint32_t M, HW, N, act;
    FastDiv dHW;
  };
  template <int MT, int NT, int FM, int FN>
  __device__ static __forceinline__ void store(const Params& p, const f4 (&acc)[FM][FN],
                                               uint32_t m0, uint32_t n0, uint32_t, int wm,
                                               int wn, int lane) {
    const int r = lane & 15, g = lane >> 4;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const uint32_t n = n0 + wn * (NT / 2) + j * 16 + r;
      const uint32_t b = fdiv(n, p.dHW);
      const uint32_t base = b * p.M * p.HW + (n - b * p.HW);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const uint32_t m = m0 + wm * (MT / 2) + i * 16 + 4 * g + v;
          if (m < p.M && n < p.N) {
            float z = acc[i][j][v];
            if (p.bias) z += p.bias[m];
            if (p.act == 1)
              z = fmaxf(z, 0.f);
            else if (p.act == 2)
              z = tanhf(z);
            p.out[base + m * p.HW] = z;
          }
        }
      }
    }
  }
};

// ---------------------------------------------------------------------------
// The kernel.
// ---------------------------------------------------------------------------
template <int MT, int NT, int KT, class LA, class LB, class EPI>
__global__ void __launch_bounds__(kThreads)
    k_igemm(const typename LA::Params pa, const typename LB::Params pb,
            const typename EPI::Params pe, uint32_t ktiles, uint32_t splits) {
  using SA = typename LA::St;
  using SB = typename LB::St;
  constexpr int WM = MT / 2, WN = NT / 2, FM = WM / 16, FN = WN / 16;
  __shared__ __attribute__((aligned(16))) float As[2 * SA::SIZE];
  __shared__ __attribute__((aligned(16))) float Bs[2 * SB::SIZE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const uint32_t m0 = blockIdx.y * MT, n0 = blockIdx.x * NT, z = blockIdx.z;
  const uint32_t kb = uint32_t((uint64_t(ktiles) * z) / splits);
  const uint32_t ke = uint32_t((uint64_t(ktiles) * (z + 1)) / splits);

  LA la;
  LB lb;
  la.init(pa, m0, tid);
  lb.init(pb, n0, tid);
  f4 ra[LA::Q], rb[LB::Q];

  f4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = zero4();

  if (kb < ke) {
    la.load(kb, ra);
    lb.load(kb, rb);
    la.store(As, ra);
    lb.store(Bs, rb);
  }
  __syncthreads();

  const int r = lane & 15, g = lane >> 4;
  for (uint32_t kt = kb; kt < ke; ++kt) {
    const int cur = int(kt - kb) & 1;
    const bool more = kt + 1 < ke;
    if (more) {
      la.load(kt + 1, ra);
      lb.load(kt + 1, rb);
    }
    const float* Ac = As + cur * SA::SIZE;
    const float* Bc = Bs + cur * SB::SIZE;
#pragma unroll
    for (int ks = 0; ks < KT; ks += 16) {
      f4 af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) af[i] = SA::frag(Ac, wm * WM + i * 16, r, g, ks);
#pragma unroll
      for (int j = 0; j < FN; ++j) bf[j] = SB::frag(Bc, wn * WN + j * 16, r, g, ks);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][s], bf[j][s], acc[i][j], 0, 0, 0);
    }
    if (more) {
      la.store(As + (cur ^ 1) * SA::SIZE, ra);
      lb.store(Bs + (cur ^ 1) * SB::SIZE, rb);
    }
    __syncthreads();
  }
  EPI::template store<MT, NT, FM, FN>(pe, acc, m0, n0, z, wm, wn, lane);
}

// ---------------------------------------------------------------------------
// Side kernels: NHWC transpose (+ ReLU mask + bias-gradient partials),
// filter re-layouts, split-K sums.
// ---------------------------------------------------------------------------
// out[((b*HW) + p)*Cp + c] = (c < C) ? in[(b*C + c)*HW + p] masked : 0.
// Block: 32 channels x 64 pixels through LDS.  dbPart[c][b*npb + block]: the
// masked values of channel c summed over the block's 64 pixels.
__global__ void __launch_bounds__(256)
    k_to_nhwc(const float* __restrict__ in, const float* __restrict__ y, float* __restrict__ out,
              float* __restrict__ dbPart, uint32_t C, uint32_t HW, uint32_t Cp, uint32_t npb) {
  __shared__ float t[32][65];
  const uint32_t c0 = blockIdx.y * 32, p0 = blockIdx.x * 64, b = blockIdx.z;
  const int tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = tid + 256 * j;
    const int cl = e >> 6, pl = e & 63;
    const uint32_t c = c0 + cl, p = p0 + pl;
    float v = 0.f;
    if (c < C && p < HW) {
      const size_t idx = (size_t(b) * C + c) * HW + p;
      v = in[idx];
      if (y != nullptr && y[idx] <= 0.f) v = 0.f;
    }
    t[cl][pl] = v;
  }
  __syncthreads();
  if (dbPart != nullptr) {
    // 8 lanes per channel, 8 pixels each, then a fixed butterfly.
    const int cl = tid >> 3, part = tid & 7;
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 8; ++q) s += t[cl][part * 8 + q];
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
    if (part == 0 && c0 + cl < C)
      dbPart[size_t(c0 + cl) * gridDim.z * npb + size_t(b) * npb + blockIdx.x] = s;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = tid + 256 * j;
    const int pl = e >> 5, cl = e & 31;
    const uint32_t c = c0 + cl, p = p0 + pl;
    if (p < HW && c < Cp) out[(size_t(b) * HW + p) * Cp + c] = t[cl][pl];
  }
}

// Few channels (Cp <= 8): one thread per output element.
__global__ void k_to_nhwc_small(const float* __restrict__ in, float* __restrict__ out, uint32_t C,
                                uint32_t HW, uint32_t Cp, uint32_t total) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const uint32_t bp = i / Cp, c = i - bp * Cp;
  const uint32_t b = bp / HW, p = bp - b * HW;
  out[i] = c < C ? in[(size_t(b) * C + c) * HW + p] : 0.f;
}

// out[c] = sum of the `rows` partials of channel c (stored contiguously,
// part[c*rows + r]): 256 strided per-thread sums, then a fixed tree.
__global__ void __launch_bounds__(256)
    k_rowsum(const float* __restrict__ part, float* __restrict__ out, uint32_t rows) {
  __shared__ float sh[4];
  const uint32_t c = blockIdx.x;
  const float* p = part + size_t(c) * rows;
  float s = 0.f;
  for (uint32_t r = threadIdx.x; r < rows; r += 256) s += p[r];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_down(s, o, 64);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) out[c] = (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

// mode 0 (forward A): out[oc][khw*Cp + c]  = c < C  ? w[oc][c][khw] : 0   (size OC*KK*Cp)
// mode 1 (dX A):      out[c][khw*OCp + oc] = oc < OC ? w[oc][c][khw] : 0  (size C*KK*OCp)
__global__ void k_permute_w(const float* __restrict__ w, float* __restrict__ out, uint32_t OC,
                            uint32_t C, uint32_t KK, uint32_t padded, int mode) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (mode == 0) {
    if (i >= OC * KK * padded) return;
    const uint32_t oc = i / (KK * padded), rr = i - oc * KK * padded;
    const uint32_t khw = rr / padded, c = rr - khw * padded;
    out[i] = c < C ? w[(oc * C + c) * KK + khw] : 0.f;
  } else {
    if (i >= C * KK * padded) return;
    const uint32_t c = i / (KK * padded), rr = i - c * KK * padded;
    const uint32_t khw = rr / padded, oc = rr - khw * padded;
    out[i] = oc < OC ? w[(oc * C + c) * KK + khw] : 0.f;
  }
}

// Deterministic split-K sum: out[i] = sum_z part[z*n + i] in z order.
__global__ void k_splitk_sum(const float* __restrict__ part, float* __restrict__ out, uint32_t n,
                             uint32_t splits) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float s = 0.f;
  for (uint32_t z = 0; z < splits; ++z) s += part[size_t(z) * n + i];
  out[i] = s;
}

// dW finalize: dw[oc][c][khw] = sum_z part[z][oc][khw*Cp + c].
__global__ void k_dw_final(const float* __restrict__ part, float* __restrict__ dw, uint32_t OC,
                           uint32_t C, uint32_t KK, uint32_t Cp, uint32_t splits) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= OC * C * KK) return;
  const uint32_t oc = i / (C * KK), rr = i - oc * C * KK;
  const uint32_t c = rr / KK, khw = rr - c * KK;
  const size_t N = size_t(KK) * Cp, src = size_t(oc) * N + khw * Cp + c, zs = size_t(OC) * N;
  float s = 0.f;
  for (uint32_t z = 0; z < splits; ++z) s += part[z * zs + src];
  dw[i] = s;
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
static int g_kt = 0;  // K-tile depth 16 (measured best); DCE_KT=32 selects 32 (tuning)
static int kt_choice() {
  if (!g_kt) {
    const char* e = getenv("DCE_KT");
    g_kt = (e && atoi(e) == 32) ? 32 : 16;
  }
  return g_kt;
}

// 128 unless 64 wastes clearly less padding.
static int pick_tile(uint32_t extent) {
  const uint64_t w128 = uint64_t(cdiv(extent, 128)) * 128, w64 = uint64_t(cdiv(extent, 64)) * 64;
  return (w128 * 100 > w64 * 112) ? 64 : 128;
}

static uint32_t pick_splits(uint32_t tiles, uint32_t ktiles, uint32_t min_kt) {
  const uint32_t target = uint32_t(num_cus()) * 2;
  if (tiles >= target) return 1;
  const uint32_t s = cdiv(target, tiles);
  const uint32_t cap = std::max<uint32_t>(1, ktiles / std::max<uint32_t>(1, min_kt));
  return std::max<uint32_t>(1, std::min(s, cap));
}

template <int MT, int NT, int KT, class LA, class LB, class EPI>
static bool launch(const typename LA::Params& pa, const typename LB::Params& pb,
                   const typename EPI::Params& pe, uint32_t M, uint32_t N, uint32_t ktiles,
                   uint32_t splits, const char* what) {
  const dim3 grid(cdiv(N, NT), cdiv(M, MT), splits);
  hipLaunchKernelGGL((k_igemm<MT, NT, KT, LA, LB, EPI>), grid, dim3(kThreads), 0, stream(), pa,
                     pb, pe, ktiles, splits);
  return check_launch(what);
}

// Dispatch a functor over the four (MT, NT) tile shapes and two KT depths.
template <class F>
static bool tiles_dispatch(int MT, int NT, int KT, F&& f) {
#define DCE_T(a, b, c) \
  if (MT == a && NT == b && KT == c) return f.template run<a, b, c>();
  DCE_T(128, 128, 32) DCE_T(128, 64, 32) DCE_T(64, 128, 32) DCE_T(64, 64, 32)
  DCE_T(128, 128, 16) DCE_T(128, 64, 16) DCE_T(64, 128, 16) DCE_T(64, 64, 16)
#undef DCE_T
  set_error("igemm: unsupported tile %dx%dx%d", MT, NT, KT);
  return false;
}

static inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// ----------------------------------------------------------------- GEMM
template <bool AT, bool BT>
struct GemmRun {
  const float *a, *b;
  float* c;
  uint32_t M, K, N, splits;
  template <int MT, int NT, int KT>
  bool run() {
    // A[m][k]: stored M×K (ROWK) or K×M (KROW); B[n][k]: stored N×K (ROWK) or K×N (KROW).
    using LA = typename std::conditional<AT, LdDenseKR<MT, KT>, LdDenseRK<MT, KT>>::type;
    using LB = typename std::conditional<BT, LdDenseRK<NT, KT>, LdDenseKR<NT, KT>>::type;
    typename LA::Params pa{a, AT ? M : K, M, K, 0};
    pa.vec = AT ? (M % 4 == 0 && aligned16(a)) : (K % 4 == 0 && aligned16(a));
    typename LB::Params pb{b, BT ? K : N, N, K, 0};
    pb.vec = BT ? (K % 4 == 0 && aligned16(b)) : (N % 4 == 0 && aligned16(b));
    EpiRowMajor::Params pe{c, M, N, N, M * N};
    return launch<MT, NT, KT, LA, LB, EpiRowMajor>(pa, pb, pe, M, N, cdiv(K, KT), splits, "gemm");
  }
};

bool gemm(const float* a, const float* b, float* c, uint32_t M, uint32_t K, uint32_t N,
          uint32_t flags) {
  if (K == 0) return fill_zero(c, size_t(M) * N);
  const int KT = kt_choice();
  const int MT = pick_tile(M), NT = pick_tile(N);
  const uint32_t tiles = cdiv(M, MT) * cdiv(N, NT);
  const uint32_t ktiles = cdiv(K, KT);
  const uint32_t splits = pick_splits(tiles, ktiles, 8);
  float* out = c;
  if (splits > 1) {
    out = workspace(size_t(splits) * M * N);
    if (!out) return false;
  }
  bool ok;
  {
    ProfScope prof("gemm", 2.0 * M * N * double(K),
                   4.0 * (double(M) * K + double(K) * N + double(M) * N));
    const bool aT = flags & 1, bT = flags & 2;
    if (!aT && !bT)
      ok = tiles_dispatch(MT, NT, KT, GemmRun<false, false>{a, b, out, M, K, N, splits});
    else if (!aT && bT)
      ok = tiles_dispatch(MT, NT, KT, GemmRun<false, true>{a, b, out, M, K, N, splits});
    else if (aT && !bT)
      ok = tiles_dispatch(MT, NT, KT, GemmRun<true, false>{a, b, out, M, K, N, splits});
    else
      ok = tiles_dispatch(MT, NT, KT, GemmRun<true, true>{a, b, out, M, K, N, splits});
  }
  if (ok && splits > 1) {
    hipLaunchKernelGGL(k_splitk_sum, dim3(cdiv(size_t(M) * N, 256)), dim3(256), 0, stream(), out,
                       c, M * N, splits);
    ok = check_launch("splitk_sum");
  }
  return ok;
}

// ----------------------------------------------------------- NHWC copies
size_t nhwc_floats(uint32_t B, uint32_t C, uint32_t H, uint32_t W) {
  return size_t(B) * H * W * pad4(C);
}

static bool to_nhwc_masked(const float* in, const float* y, float* out, float* dbPart,
                           uint32_t B, uint32_t C, uint32_t HW, uint32_t* npbOut) {
  const uint32_t Cp = pad4(C);
  if (Cp <= 8 && !y && !dbPart) {
    const size_t total = size_t(B) * HW * Cp;
    hipLaunchKernelGGL(k_to_nhwc_small, dim3(cdiv(total, 256)), dim3(256), 0, stream(), in, out,
                       C, HW, Cp, uint32_t(total));
    return check_launch("to_nhwc");
  }
  const uint32_t npb = cdiv(HW, 64);
  if (npbOut) *npbOut = npb;
  hipLaunchKernelGGL(k_to_nhwc, dim3(npb, cdiv(Cp, 32), B), dim3(256), 0, stream(), in, y, out,
                     dbPart, C, HW, Cp, npb);
  return check_launch("to_nhwc");
}

bool to_nhwc(const float* x, float* out, uint32_t B, uint32_t C, uint32_t H, uint32_t W) {
  return to_nhwc_masked(x, nullptr, out, nullptr, B, C, H * W, nullptr);
}

// ----------------------------------------------------------- conv forward
template <bool S1>
struct FwdRun {
  const float* wp;
  const float* xn;
  const float* bias;
  float* y;
  ConvGeom g;
  uint32_t act;
  template <int MT, int NT, int KT>
  bool run() {
    const uint32_t Cp = pad4(g.C), KK = g.k * g.k, kdim = KK * Cp;
    const uint32_t OHW = g.OH * g.OW, N = g.B * OHW;
    using LA = LdDenseRK<MT, KT>;
    using LB = LdPixRK<NT, KT, true, S1>;
    typename LA::Params pa{wp, kdim, g.OC, kdim, 1};
    typename LB::Params pb{xn, g.H, g.W, Cp, g.k, g.s, g.p, g.OW, OHW, N, kdim,
                           make_fastdiv(OHW), make_fastdiv(g.OW), make_fastdiv(Cp), make_fastdiv(g.k)};
    EpiNCHW::Params pe{y, bias, g.OC, OHW, N, act, make_fastdiv(OHW)};
    return launch<MT, NT, KT, LA, LB, EpiNCHW>(pa, pb, pe, g.OC, N, cdiv(kdim, KT), 1,
                                              "conv_forward");
  }
};

bool conv_forward(const float* x, float* x_nhwc_keep, const float* w, const float* bias,
                  float* y, const ConvGeom& g, uint32_t act) {
  const uint32_t Cp = pad4(g.C), KK = g.k * g.k;
  const size_t nx = nhwc_floats(g.B, g.C, g.H, g.W);
  const size_t nw = (size_t(g.OC) * KK * Cp + 63) & ~size_t(63);
  float* ws = workspace(nw + (x_nhwc_keep ? 0 : nx));
  if (!ws) return false;
  float* wp = ws;
  float* xn = x_nhwc_keep ? x_nhwc_keep : ws + nw;
  if (!to_nhwc(x, xn, g.B, g.C, g.H, g.W)) return false;
  hipLaunchKernelGGL(k_permute_w, dim3(cdiv(size_t(g.OC) * KK * Cp, 256)), dim3(256), 0, stream(),
                     w, wp, g.OC, g.C, KK, Cp, 0);
  if (!check_launch("permute_w")) return false;
  const double fl = 2.0 * g.OC * g.C * KK * double(g.B) * g.OH * g.OW;
  ProfScope prof("conv_fwd", fl,
                 4.0 * (double(g.B) * g.C * g.H * g.W + double(g.B) * g.OC * g.OH * g.OW));
  const int MT = pick_tile(g.OC), NT = 128, KT = kt_choice();
  if (g.s == 1) return tiles_dispatch(MT, NT, KT, FwdRun<true>{wp, xn, bias, y, g, act});
  return tiles_dispatch(MT, NT, KT, FwdRun<false>{wp, xn, bias, y, g, act});
}

// ----------------------------------------------------------- conv backward
struct DwRun {
  const float* gn;
  const float* xn;
  float* part;
  ConvGeom g;
  uint32_t splits;
  template <int MT, int NT, int KT>
  bool run() {
    const uint32_t Cp = pad4(g.C), OCp = pad4(g.OC), KK = g.k * g.k, N = KK * Cp;
    const uint32_t OHW = g.OH * g.OW, npix = g.B * OHW;
    using LA = LdGradKR<MT, KT>;
    using LB = LdXTapKR<NT, KT>;
    typename LA::Params pa{gn, OCp, npix};
    typename LB::Params pb{xn, g.H, g.W, Cp, g.k, g.s, g.p, g.OW, OHW, npix, N,
                           make_fastdiv(OHW), make_fastdiv(g.OW), make_fastdiv(Cp), make_fastdiv(g.k)};
    EpiRowMajor::Params pe{part, g.OC, N, N, g.OC * N};
    return launch<MT, NT, KT, LA, LB, EpiRowMajor>(pa, pb, pe, g.OC, N, cdiv(npix, KT), splits,
                                                  "conv_backward_filter");
  }
};

template <bool S1>
struct DxRun {
  const float* wt;
  const float* gn;
  float* dx;
  ConvGeom g;
  template <int MT, int NT, int KT>
  bool run() {
    const uint32_t OCp = pad4(g.OC), KK = g.k * g.k, kdim = KK * OCp;
    const uint32_t HW = g.H * g.W, N = g.B * HW;
    using LA = LdDenseRK<MT, KT>;
    using LB = LdPixRK<NT, KT, false, S1>;
    typename LA::Params pa{wt, kdim, g.C, kdim, 1};
    typename LB::Params pb{gn, g.OH, g.OW, OCp, g.k, g.s, g.p, g.W, HW, N, kdim,
                           make_fastdiv(HW), make_fastdiv(g.W), make_fastdiv(OCp), make_fastdiv(g.k)};
    EpiNCHW::Params pe{dx, nullptr, g.C, HW, N, 0, make_fastdiv(HW)};
    return launch<MT, NT, KT, LA, LB, EpiNCHW>(pa, pb, pe, g.C, N, cdiv(kdim, KT), 1,
                                              "conv_backward_input");
  }
};

static inline size_t al64(size_t n) { return (n + 63) & ~size_t(63); }

bool conv_backward(const float* dy, const float* y, const float* x, const float* x_nhwc,
                   const float* w, float* dw, float* db, float* dx, const ConvGeom& g) {
  const uint32_t Cp = pad4(g.C), OCp = pad4(g.OC), KK = g.k * g.k;
  const uint32_t OHW = g.OH * g.OW, npix = g.B * OHW;
  const int KT = kt_choice();
  // Workspace carve-up: G (NHWC), db partials, x (NHWC) if not kept by the
  // forward, dW split-K partials, dX filters.
  const uint32_t npb = cdiv(OHW, 64);
  const size_t nG = al64(size_t(npix) * OCp);
  const size_t nDb = db ? al64(size_t(g.B) * npb * g.OC) : 0;
  const size_t nX = (dw && !x_nhwc) ? al64(nhwc_floats(g.B, g.C, g.H, g.W)) : 0;
  int dMT = 128, dNT = 128;
  uint32_t splits = 1;
  size_t nP = 0;
  if (dw) {
    dMT = pick_tile(g.OC);
    dNT = pick_tile(KK * Cp);
    const uint32_t tiles = cdiv(g.OC, dMT) * cdiv(KK * Cp, dNT);
    splits = pick_splits(tiles, cdiv(npix, KT), 8);
    nP = al64(size_t(splits) * g.OC * KK * Cp);
  }
  const size_t nW = dx ? al64(size_t(g.C) * KK * OCp) : 0;
  float* ws = workspace(nG + nDb + nX + nP + nW);
  if (!ws) return false;
  float* gn = ws;
  float* dbPart = db ? gn + nG : nullptr;
  float* xs = ws + nG + nDb;
  float* part = xs + nX;
  float* wt = part + nP;

  uint32_t npbGot = npb;
  if (!to_nhwc_masked(dy, y, gn, dbPart, g.B, g.OC, OHW, &npbGot)) return false;
  if (db) {
    hipLaunchKernelGGL(k_rowsum, dim3(g.OC), dim3(256), 0, stream(), dbPart, db, g.B * npb);
    if (!check_launch("bias_grad")) return false;
  }
  if (dw) {
    const float* xn = x_nhwc;
    if (!xn) {
      if (!to_nhwc(x, xs, g.B, g.C, g.H, g.W)) return false;
      xn = xs;
    }
    bool ok;
    {
      const double fl = 2.0 * g.OC * g.C * KK * double(npix);
      ProfScope prof("conv_dw", fl,
                     4.0 * (double(npix) * OCp + double(g.B) * g.H * g.W * Cp + double(g.OC) * KK * Cp));
      ok = tiles_dispatch(dMT, dNT, KT, DwRun{gn, xn, part, g, splits});
    }
    if (!ok) return false;
    hipLaunchKernelGGL(k_dw_final, dim3(cdiv(size_t(g.OC) * g.C * KK, 256)), dim3(256), 0,
                       stream(), part, dw, g.OC, g.C, KK, Cp, splits);
    if (!check_launch("dw_final")) return false;
  }
  if (dx) {
    hipLaunchKernelGGL(k_permute_w, dim3(cdiv(size_t(g.C) * KK * OCp, 256)), dim3(256), 0,
                       stream(), w, wt, g.OC, g.C, KK, OCp, 1);
    if (!check_launch("permute_w")) return false;
    const double fl = 2.0 * g.OC * g.C * KK * double(npix);
    ProfScope prof("conv_dx", fl, 4.0 * (double(npix) * OCp + double(g.B) * g.C * g.H * g.W));
    const int MT = pick_tile(g.C), NT = 128;
    if (g.s == 1) return tiles_dispatch(MT, NT, KT, DxRun<true>{wt, gn, dx, g});
    return tiles_dispatch(MT, NT, KT, DxRun<false>{wt, gn, dx, g});
  }
  return true;
}

}  // namespace dce
