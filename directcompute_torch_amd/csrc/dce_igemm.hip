// fp32 implicit-GEMM on CDNA4 matrix cores (v_mfma_f32_16x16x4_f32) for the
// convolution forward, filter gradient (dW + fused db), input gradient (dX)
// and the flagged dense GEMM of MatMulAlloc.
//
// One kernel template, four operand loaders and three epilogues:
//
//   C[m, n] = sum_k A[m, k] * B[n, k]
//
//   * 256 threads = 4 wave64 in a 2x2 arrangement; a workgroup owns an
//     MT x NT output tile (MT, NT in {64, 128}); each wave an (MT/2) x (NT/2)
//     block of 16x16 MFMA accumulators.
//   * K advances in tiles of KT = 16.  Both operands are staged in LDS as
//     [row][k] with a row stride of KT + 4 floats; every thread fetches whole
//     k-quads (4 consecutive k of one row) from global memory into registers
//     one tile ahead, then writes them with one ds_write_b128 into the other
//     half of a double buffer -- one barrier per k-tile.
//   * MFMA operands are read with ds_read_b128: in the 4 MFMAs of a 16-wide
//     k slice, lane l (r = l % 16, g = l / 16) supplies A[r][4g + s] and
//     B[4g + s][r] in MFMA s, so the four instructions together cover k
//     0..15 (the matrix unit sums over g, the loop over s).  With the +4
//     padding, 8 consecutive lanes hit 32 distinct banks.
//   * Split-K over blockIdx.z writes partial tiles that a deterministic
//     second pass sums in a fixed order (no atomics).
//
// The loaders turn a (row, k-quad) into addresses of the real tensors, so no
// im2col / col2im / reshaped-gradient buffer is ever materialised:
//   DenseLoader  : plain matrix, row-major or k-major (GEMM operands, filters)
//   GLoader      : dW "A" = ReLU-masked dy rows (oc) over k = (image, pixel)
//                  + the bias-gradient row sums, accumulated from registers
//   XColLoader   : dW "B" = x patches, rows (c, kh, kw) over k = (image, pixel)
//   XPixLoader   : forward "B" = x patches, rows = output pixels
//   GPixLoader   : dX "B" = masked dy patches, rows = input pixels
#include "dce_internal.h"

#include <algorithm>

namespace dce {

typedef float f4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int KT = 16;
constexpr int LDK = KT + 4;
constexpr int KQ = KT / 4;

// Thread -> (row, k-quad) assignment.  ROWFAST: consecutive lanes take
// consecutive rows (for operands contiguous along the row index); otherwise
// consecutive lanes take consecutive k-quads of one row.
template <int R, bool ROWFAST>
struct QMap {
  static_assert((R * KQ) % kThreads == 0, "tile rows must fill the workgroup");
  static constexpr int Q = R * KQ / kThreads;
  __device__ static __forceinline__ int row(int tid, int i) {
    int q = tid + kThreads * i;
    return ROWFAST ? (q % R) : (q / KQ);
  }
  __device__ static __forceinline__ int kq(int tid, int i) {
    int q = tid + kThreads * i;
    return ROWFAST ? (q / R) : (q % KQ);
  }
};

template <int R, bool ROWFAST>
struct LoaderBase {
  using Map = QMap<R, ROWFAST>;
  static constexpr int Q = Map::Q;
  int lds_off[Q];
  int kqi[Q];
  __device__ __forceinline__ void base_init(int tid) {
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      kqi[i] = Map::kq(tid, i);
      lds_off[i] = Map::row(tid, i) * LDK + 4 * kqi[i];
    }
  }
  __device__ __forceinline__ void store(float* lds, const f4 (&r)[Q]) const {
#pragma unroll
    for (int i = 0; i < Q; ++i) *reinterpret_cast<f4*>(lds + lds_off[i]) = r[i];
  }
  __device__ __forceinline__ void finish(uint32_t) const {}
};

// ---------------------------------------------------------------------------
// DenseLoader: element (row, k) of a matrix stored row-major ([row][k], ld =
// row pitch) or k-major ([k][row], ld = k pitch).
// ---------------------------------------------------------------------------
template <int R, bool KMAJOR>
struct DenseLoader : LoaderBase<R, KMAJOR> {
  using Base = LoaderBase<R, KMAJOR>;
  using Base::Q;
  using Base::kqi;
  struct Params {
    const float* ptr;
    uint32_t ld, rows, kdim, vec4;
  };
  const float* ptr;
  uint32_t ld, kdim;
  bool vec;
  uint32_t rowi[Q];
  bool rok[Q];

  __device__ __forceinline__ void init(const Params& p, uint32_t row0, int tid) {
    this->base_init(tid);
    ptr = p.ptr;
    ld = p.ld;
    kdim = p.kdim;
    vec = p.vec4 != 0;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      rowi[i] = row0 + Base::Map::row(tid, i);
      rok[i] = rowi[i] < p.rows;
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) {
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t k0 = kt * KT + 4 * kqi[i];
      if (KMAJOR) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t k = k0 + e;
          r[i][e] = (rok[i] && k < kdim) ? ptr[k * ld + rowi[i]] : 0.f;
        }
      } else if (vec) {
        f4 z = {0.f, 0.f, 0.f, 0.f};
        r[i] = (rok[i] && k0 < kdim) ? *reinterpret_cast<const f4*>(ptr + rowi[i] * ld + k0) : z;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t k = k0 + e;
          r[i][e] = (rok[i] && k < kdim) ? ptr[rowi[i] * ld + k] : 0.f;
        }
      }
    }
  }
};

// ---------------------------------------------------------------------------
// GLoader (dW operand A): A[oc][k], k = (image b, pixel), value dy masked by
// the ReLU output (y <= 0 -> 0, engine semantics of conv_grad_reshape_relu).
// k-tiles run over (b, pixel chunk of KT); the last chunk of an image is
// partial.  Row sums of A (= the bias gradient) are accumulated from the
// loaded registers by the workgroups of the first n-tile.
// ---------------------------------------------------------------------------
template <int R>
struct GLoader : LoaderBase<R, false> {
  using Base = LoaderBase<R, false>;
  using Base::Q;
  using Base::kqi;
  struct Params {
    const float* dy;
    const float* y;
    float* dbPart;  // [splits][OC] or null
    uint32_t OC, OHW, nchunk;
    FastDiv dChunk;
  };
  const float* dy;
  const float* y;
  uint32_t OHW, nchunk, img;
  FastDiv dChunk;
  uint32_t rowoff[Q];
  bool rok[Q];
  float rsum[Q];
  bool doSum;
  float* dbPart;
  uint32_t OC;
  uint32_t ocv[Q];

  __device__ __forceinline__ void init(const Params& p, uint32_t row0, int tid) {
    this->base_init(tid);
    dy = p.dy;
    y = p.y;
    OHW = p.OHW;
    nchunk = p.nchunk;
    dChunk = p.dChunk;
    img = p.OC * p.OHW;
    OC = p.OC;
    dbPart = p.dbPart;
    doSum = p.dbPart != nullptr && blockIdx.x == 0;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      ocv[i] = row0 + Base::Map::row(tid, i);
      rok[i] = ocv[i] < p.OC;
      rowoff[i] = ocv[i] * p.OHW;
      rsum[i] = 0.f;
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) {
    const uint32_t b = fdiv(kt, dChunk);
    const uint32_t ch = kt - b * nchunk;
    const uint32_t base = b * img;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t pix0 = ch * KT + 4 * kqi[i];
      const uint32_t off = base + rowoff[i] + pix0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool valid = rok[i] && (pix0 + e) < OHW;
        float v = valid ? dy[off + e] : 0.f;
        if (y != nullptr && valid) {
          if (y[off + e] <= 0.f) v = 0.f;
        }
        r[i][e] = v;
      }
      if (doSum) rsum[i] += (r[i][0] + r[i][1]) + (r[i][2] + r[i][3]);
    }
  }
  __device__ __forceinline__ void finish(uint32_t z) {
    if (dbPart == nullptr || blockIdx.x != 0) return;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      float s = rsum[i];
      // The KQ lanes holding one row are consecutive: butterfly over them.
#pragma unroll
      for (int o = 1; o < KQ; o <<= 1) s += __shfl_xor(s, o, 64);
      if (kqi[i] == 0 && rok[i]) dbPart[z * OC + ocv[i]] = s;
    }
  }
};

// ---------------------------------------------------------------------------
// XColLoader (dW operand B): B[n][k], n = (c, kh, kw), k = (image b, pixel
// (oh, ow)) -> x[b, c, oh*s + kh - p, ow*s + kw - p] or 0.
// ---------------------------------------------------------------------------
template <int R>
struct XColLoader : LoaderBase<R, false> {
  using Base = LoaderBase<R, false>;
  using Base::Q;
  using Base::kqi;
  struct Params {
    const float* x;
    uint32_t C, H, W, k, s, p, OW, OHW, nchunk, N;
    FastDiv dOW, dK, dKK, dChunk;
  };
  const float* x;
  uint32_t H, W, s, OW, OHW, nchunk, img;
  FastDiv dOW, dChunk;
  uint32_t coff[Q];
  int ihb[Q], iwb[Q];
  bool rok[Q];

  __device__ __forceinline__ void init(const Params& p, uint32_t row0, int tid) {
    this->base_init(tid);
    x = p.x;
    H = p.H;
    W = p.W;
    s = p.s;
    OW = p.OW;
    OHW = p.OHW;
    nchunk = p.nchunk;
    img = p.C * p.H * p.W;
    dOW = p.dOW;
    dChunk = p.dChunk;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t n = row0 + Base::Map::row(tid, i);
      rok[i] = n < p.N;
      const uint32_t c = fdiv(n, p.dKK);
      const uint32_t rr = n - c * p.k * p.k;
      const uint32_t kh = fdiv(rr, p.dK);
      const uint32_t kw = rr - kh * p.k;
      coff[i] = c * p.H * p.W;
      ihb[i] = int(kh) - int(p.p);
      iwb[i] = int(kw) - int(p.p);
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) {
    const uint32_t b = fdiv(kt, dChunk);
    const uint32_t ch = kt - b * nchunk;
    const uint32_t xb = b * img;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t pix0 = ch * KT + 4 * kqi[i];
      uint32_t oh = fdiv(pix0, dOW);
      uint32_t ow = pix0 - oh * OW;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int ih = int(oh * s) + ihb[i];
        const int iw = int(ow * s) + iwb[i];
        const bool valid = rok[i] && (pix0 + e) < OHW && uint32_t(ih) < H && uint32_t(iw) < W;
        r[i][e] = valid ? x[xb + coff[i] + uint32_t(ih) * W + uint32_t(iw)] : 0.f;
        if (++ow == OW) {
          ow = 0;
          ++oh;
        }
      }
    }
  }
};

// ---------------------------------------------------------------------------
// XPixLoader (forward operand B): B[n][k], n = output pixel (b, oh, ow),
// k = (kh, kw, c) in channel chunks of KT (CHUNK, needs C % KT == 0) or flat
// (c, kh, kw) otherwise; value x[b, c, oh*s + kh - p, ow*s + kw - p] or 0.
// ---------------------------------------------------------------------------
template <int R, bool CHUNK>
struct XPixLoader : LoaderBase<R, true> {
  using Base = LoaderBase<R, true>;
  using Base::Q;
  using Base::kqi;
  struct Params {
    const float* x;
    uint32_t C, H, W, k, s, p, OW, OHW, N, kdim, nch;
    FastDiv dOHW, dOW, dK, dKK, dNch;
  };
  const float* x;
  uint32_t C, H, W, k, HW, kdim, nch;
  FastDiv dK, dKK, dNch;
  uint32_t xoff[Q];
  int ih0[Q], iw0[Q];
  bool rok[Q];

  __device__ __forceinline__ void init(const Params& p, uint32_t row0, int tid) {
    this->base_init(tid);
    x = p.x;
    C = p.C;
    H = p.H;
    W = p.W;
    k = p.k;
    HW = p.H * p.W;
    kdim = p.kdim;
    nch = p.nch;
    dK = p.dK;
    dKK = p.dKK;
    dNch = p.dNch;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t n = row0 + Base::Map::row(tid, i);
      rok[i] = n < p.N;
      const uint32_t b = fdiv(n, p.dOHW);
      const uint32_t pix = n - b * p.OHW;
      const uint32_t oh = fdiv(pix, p.dOW);
      const uint32_t ow = pix - oh * p.OW;
      xoff[i] = b * p.C * HW;
      ih0[i] = int(oh * p.s) - int(p.p);
      iw0[i] = int(ow * p.s) - int(p.p);
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) {
    if (CHUNK) {
      const uint32_t khw = fdiv(kt, dNch);
      const uint32_t cc = kt - khw * nch;
      const uint32_t kh = fdiv(khw, dK);
      const uint32_t kw = khw - kh * k;
#pragma unroll
      for (int i = 0; i < Q; ++i) {
        const int ih = ih0[i] + int(kh);
        const int iw = iw0[i] + int(kw);
        const bool valid = rok[i] && uint32_t(ih) < H && uint32_t(iw) < W;
        const uint32_t c0 = cc * KT + 4 * kqi[i];
        const uint32_t base = xoff[i] + c0 * HW + uint32_t(ih) * W + uint32_t(iw);
#pragma unroll
        for (int e = 0; e < 4; ++e) r[i][e] = (valid && c0 + e < C) ? x[base + e * HW] : 0.f;
      }
    } else {
#pragma unroll
      for (int i = 0; i < Q; ++i) {
        const uint32_t kk0 = kt * KT + 4 * kqi[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t kk = kk0 + e;
          const uint32_t c = fdiv(kk, dKK);
          const uint32_t rr = kk - c * k * k;
          const uint32_t kh = fdiv(rr, dK);
          const uint32_t kw = rr - kh * k;
          const int ih = ih0[i] + int(kh);
          const int iw = iw0[i] + int(kw);
          const bool valid = rok[i] && kk < kdim && uint32_t(ih) < H && uint32_t(iw) < W;
          r[i][e] = valid ? x[xoff[i] + c * HW + uint32_t(ih) * W + uint32_t(iw)] : 0.f;
        }
      }
    }
  }
};

// ---------------------------------------------------------------------------
// GPixLoader (dX operand B): B[n][k], n = input pixel (b, ih, iw), k = (kh,
// kw, oc) in oc chunks of KT (CHUNK, needs OC % KT == 0) or flat (oc, kh, kw);
// value = masked dy[b, oc, oh, ow] where oh*s = ih + p - kh exactly (C-style
// divisibility as col2im) and in range, else 0.
// ---------------------------------------------------------------------------
template <int R, bool CHUNK, bool S1>
struct GPixLoader : LoaderBase<R, true> {
  using Base = LoaderBase<R, true>;
  using Base::Q;
  using Base::kqi;
  struct Params {
    const float* dy;
    const float* y;
    uint32_t OC, H, W, k, s, p, OH, OW, N, kdim, noc;
    FastDiv dHW, dW, dK, dKK, dNoc;
  };
  const float* dy;
  const float* y;
  uint32_t OC, k, s, OH, OW, OHW, kdim, noc;
  FastDiv dK, dKK, dNoc;
  uint32_t goff[Q];
  int ihp[Q], iwp[Q];
  bool rok[Q];

  __device__ __forceinline__ void init(const Params& p, uint32_t row0, int tid) {
    this->base_init(tid);
    dy = p.dy;
    y = p.y;
    OC = p.OC;
    k = p.k;
    s = p.s;
    OH = p.OH;
    OW = p.OW;
    OHW = p.OH * p.OW;
    kdim = p.kdim;
    noc = p.noc;
    dK = p.dK;
    dKK = p.dKK;
    dNoc = p.dNoc;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t n = row0 + Base::Map::row(tid, i);
      rok[i] = n < p.N;
      const uint32_t b = fdiv(n, p.dHW);
      const uint32_t pix = n - b * p.H * p.W;
      const uint32_t ih = fdiv(pix, p.dW);
      const uint32_t iw = pix - ih * p.W;
      goff[i] = b * p.OC * OHW;
      ihp[i] = int(ih + p.p);
      iwp[i] = int(iw + p.p);
    }
  }
  __device__ __forceinline__ bool tap(int i, uint32_t kh, uint32_t kw, uint32_t& sp) const {
    const int oh_s = ihp[i] - int(kh);
    const int ow_s = iwp[i] - int(kw);
    if (S1) {
      sp = uint32_t(oh_s) * OW + uint32_t(ow_s);
      return rok[i] && uint32_t(oh_s) < OH && uint32_t(ow_s) < OW;
    }
    if (oh_s < 0 || ow_s < 0) return false;
    const uint32_t oh = uint32_t(oh_s) / s, ow = uint32_t(ow_s) / s;
    sp = oh * OW + ow;
    return rok[i] && oh * s == uint32_t(oh_s) && ow * s == uint32_t(ow_s) && oh < OH && ow < OW;
  }
  __device__ __forceinline__ float fetch(uint32_t off) const {
    float v = dy[off];
    if (y != nullptr && y[off] <= 0.f) v = 0.f;
    return v;
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) {
    if (CHUNK) {
      const uint32_t khw = fdiv(kt, dNoc);
      const uint32_t occ = kt - khw * noc;
      const uint32_t kh = fdiv(khw, dK);
      const uint32_t kw = khw - kh * k;
#pragma unroll
      for (int i = 0; i < Q; ++i) {
        uint32_t sp = 0;
        const bool valid = tap(i, kh, kw, sp);
        const uint32_t oc0 = occ * KT + 4 * kqi[i];
        const uint32_t base = goff[i] + oc0 * OHW + sp;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[i][e] = (valid && oc0 + e < OC) ? fetch(base + e * OHW) : 0.f;
      }
    } else {
#pragma unroll
      for (int i = 0; i < Q; ++i) {
        const uint32_t kk0 = kt * KT + 4 * kqi[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t kk = kk0 + e;
          const uint32_t oc = fdiv(kk, dKK);
          const uint32_t rr = kk - oc * k * k;
          const uint32_t kh = fdiv(rr, dK);
          const uint32_t kw = rr - kh * k;
          uint32_t sp = 0;
          const bool valid = kk < kdim && tap(i, kh, kw, sp);
          r[i][e] = valid ? fetch(goff[i] + oc * OHW + sp) : 0.f;
        }
      }
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

struct EpiConvFwd {
  struct Params {
    float* y;
    const float* bias;
    uint32_t OC, OHW, N, act;
    FastDiv dOHW;
  };
  template <int MT, int NT, int FM, int FN>
  __device__ static __forceinline__ void store(const Params& p, const f4 (&acc)[FM][FN],
                                               uint32_t m0, uint32_t n0, uint32_t, int wm,
                                               int wn, int lane) {
    const int r = lane & 15, g = lane >> 4;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const uint32_t n = n0 + wn * (NT / 2) + j * 16 + r;
      const uint32_t b = fdiv(n, p.dOHW);
      const uint32_t base = b * p.OC * p.OHW + (n - b * p.OHW);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const uint32_t m = m0 + wm * (MT / 2) + i * 16 + 4 * g + v;
          if (m < p.OC && n < p.N) {
            float z = acc[i][j][v] + p.bias[m];
            if (p.act == 1)
              z = fmaxf(z, 0.f);
            else if (p.act == 2)
              z = tanhf(z);
            p.y[base + m * p.OHW] = z;
          }
        }
      }
    }
  }
};

struct EpiConvDx {
  struct Params {
    float* dx;
    uint32_t C, HW, N;
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
      const uint32_t base = b * p.C * p.HW + (n - b * p.HW);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const uint32_t m = m0 + wm * (MT / 2) + i * 16 + 4 * g + v;
          if (m < p.C && n < p.N) p.dx[base + m * p.HW] = acc[i][j][v];
        }
      }
    }
  }
};

// ---------------------------------------------------------------------------
// The kernel.
// ---------------------------------------------------------------------------
template <int MT, int NT, class LA, class LB, class EPI>
__global__ void __launch_bounds__(kThreads)
    k_igemm(const typename LA::Params pa, const typename LB::Params pb,
            const typename EPI::Params pe, uint32_t ktiles, uint32_t splits) {
  constexpr int WM = MT / 2, WN = NT / 2, FM = WM / 16, FN = WN / 16;
  __shared__ __attribute__((aligned(16))) float As[2 * MT * LDK];
  __shared__ __attribute__((aligned(16))) float Bs[2 * NT * LDK];

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
    for (int j = 0; j < FN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  if (kb < ke) {
    la.load(kb, ra);
    lb.load(kb, rb);
    la.store(As, ra);
    lb.store(Bs, rb);
  }
  __syncthreads();

  const int r = lane & 15, g = lane >> 4;
  const int aoff = (wm * WM + r) * LDK + 4 * g;
  const int boff = (wn * WN + r) * LDK + 4 * g;

  for (uint32_t kt = kb; kt < ke; ++kt) {
    const int cur = int(kt - kb) & 1;
    const bool more = kt + 1 < ke;
    if (more) {
      la.load(kt + 1, ra);
      lb.load(kt + 1, rb);
    }
    const float* Ac = As + cur * (MT * LDK);
    const float* Bc = Bs + cur * (NT * LDK);
    f4 af[FM], bf[FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) af[i] = *reinterpret_cast<const f4*>(Ac + aoff + i * 16 * LDK);
#pragma unroll
    for (int j = 0; j < FN; ++j) bf[j] = *reinterpret_cast<const f4*>(Bc + boff + j * 16 * LDK);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][s], bf[j][s], acc[i][j], 0, 0, 0);
    if (more) {
      la.store(As + (cur ^ 1) * (MT * LDK), ra);
      lb.store(Bs + (cur ^ 1) * (NT * LDK), rb);
    }
    __syncthreads();
  }
  EPI::template store<MT, NT, FM, FN>(pe, acc, m0, n0, z, wm, wn, lane);
  la.finish(z);
}

// Deterministic split-K sum: out[i] = sum_z part[z*n + i] in z order.
__global__ void k_splitk_sum(const float* __restrict__ part, float* __restrict__ out,
                             uint32_t n, uint32_t splits) {
  uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float s = 0.f;
  for (uint32_t z = 0; z < splits; ++z) s += part[size_t(z) * n + i];
  out[i] = s;
}

// Filter re-layouts for the conv GEMM A operands (tiny tensors).
//  mode 0 (forward, channel chunks): out[oc][khw][c]
//  mode 1 (dX, oc chunks):           out[c][khw][oc]
//  mode 2 (dX, flat):                out[c][oc][khw]
__global__ void k_permute_w(const float* __restrict__ w, float* __restrict__ out, uint32_t OC,
                            uint32_t C, uint32_t KK, int mode) {
  uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t n = OC * C * KK;
  if (i >= n) return;
  uint32_t oc = i / (C * KK);
  uint32_t rr = i - oc * C * KK;
  uint32_t c = rr / KK;
  uint32_t khw = rr - c * KK;
  uint32_t d;
  if (mode == 0)
    d = (oc * KK + khw) * C + c;
  else if (mode == 1)
    d = (c * KK + khw) * OC + oc;
  else
    d = (c * OC + oc) * KK + khw;
  out[d] = w[i];
}

// ---------------------------------------------------------------------------
// Host side: tile choice, split-K, launches.
// ---------------------------------------------------------------------------
static inline uint32_t cdiv(uint64_t a, uint64_t b) { return uint32_t((a + b - 1) / b); }

// 128 unless 64 wastes clearly less padding.
static int pick_tile(uint32_t extent) {
  uint64_t w128 = uint64_t(cdiv(extent, 128)) * 128, w64 = uint64_t(cdiv(extent, 64)) * 64;
  return (w128 * 100 > w64 * 112) ? 64 : 128;
}

template <int MT, int NT, class LA, class LB, class EPI>
static bool launch(const typename LA::Params& pa, const typename LB::Params& pb,
                   const typename EPI::Params& pe, uint32_t M, uint32_t N, uint32_t ktiles,
                   uint32_t splits, const char* what) {
  dim3 grid(cdiv(N, NT), cdiv(M, MT), splits);
  hipLaunchKernelGGL((k_igemm<MT, NT, LA, LB, EPI>), grid, dim3(kThreads), 0, stream(), pa, pb,
                     pe, ktiles, splits);
  return check_launch(what);
}

static uint32_t pick_splits(uint32_t tiles, uint32_t ktiles, uint32_t min_kt) {
  const uint32_t target = uint32_t(num_cus()) * 2;
  if (tiles >= target) return 1;
  uint32_t s = cdiv(target, tiles);
  uint32_t cap = std::max<uint32_t>(1, ktiles / std::max<uint32_t>(1, min_kt));
  return std::max<uint32_t>(1, std::min(s, cap));
}

static bool splitk_sum(const float* part, float* out, uint32_t n, uint32_t splits) {
  hipLaunchKernelGGL(k_splitk_sum, dim3(cdiv(n, 256)), dim3(256), 0, stream(), part, out, n,
                     splits);
  return check_launch("splitk_sum");
}

// ----------------------------------------------------------------- GEMM
template <int MT, int NT, bool AK, bool BK>
static bool gemm_tiles(const float* a, const float* b, float* c, uint32_t M, uint32_t K,
                       uint32_t N, float* part, uint32_t splits) {
  using LA = DenseLoader<MT, AK>;
  using LB = DenseLoader<NT, BK>;
  typename LA::Params pa{a, AK ? M : K, M, K, 0};
  typename LB::Params pb{b, BK ? N : K, N, K, 0};
  if (!AK) pa.vec4 = (K % 4 == 0 && (reinterpret_cast<uintptr_t>(a) & 15) == 0);
  if (!BK) pb.vec4 = (K % 4 == 0 && (reinterpret_cast<uintptr_t>(b) & 15) == 0);
  EpiRowMajor::Params pe{splits > 1 ? part : c, M, N, N, M * N};
  return launch<MT, NT, LA, LB, EpiRowMajor>(pa, pb, pe, M, N, cdiv(K, KT), splits, "gemm");
}

template <bool AK, bool BK>
static bool gemm_flags(const float* a, const float* b, float* c, uint32_t M, uint32_t K,
                       uint32_t N, float* part, uint32_t splits, int MT, int NT) {
  if (MT == 128 && NT == 128) return gemm_tiles<128, 128, AK, BK>(a, b, c, M, K, N, part, splits);
  if (MT == 128) return gemm_tiles<128, 64, AK, BK>(a, b, c, M, K, N, part, splits);
  if (NT == 128) return gemm_tiles<64, 128, AK, BK>(a, b, c, M, K, N, part, splits);
  return gemm_tiles<64, 64, AK, BK>(a, b, c, M, K, N, part, splits);
}

bool gemm(const float* a, const float* b, float* c, uint32_t M, uint32_t K, uint32_t N,
          uint32_t flags) {
  if (K == 0) return fill_zero(c, size_t(M) * N);
  const int MT = pick_tile(M), NT = pick_tile(N);
  const uint32_t tiles = cdiv(M, MT) * cdiv(N, NT);
  const uint32_t ktiles = cdiv(K, KT);
  uint32_t splits = pick_splits(tiles, ktiles, 8);
  float* part = nullptr;
  if (splits > 1) {
    part = workspace(size_t(splits) * M * N);
    if (!part) return false;
  }
  ProfScope prof("gemm", 2.0 * M * N * double(K), 4.0 * (double(M) * K + double(K) * N + double(M) * N));
  const bool aK = flags & 1, bN = !(flags & 2);  // A k-major if transposed; B row-fast if not
  bool ok;
  if (!aK && !bN)
    ok = gemm_flags<false, false>(a, b, c, M, K, N, part, splits, MT, NT);
  else if (!aK && bN)
    ok = gemm_flags<false, true>(a, b, c, M, K, N, part, splits, MT, NT);
  else if (aK && !bN)
    ok = gemm_flags<true, false>(a, b, c, M, K, N, part, splits, MT, NT);
  else
    ok = gemm_flags<true, true>(a, b, c, M, K, N, part, splits, MT, NT);
  if (ok && splits > 1) ok = splitk_sum(part, c, M * N, splits);
  return ok;
}

// ----------------------------------------------------------- conv forward
template <int MT, bool CHUNK>
static bool conv_fwd_t(const float* x, const float* wA, const float* bias, float* y,
                       const ConvGeom& g, uint32_t act) {
  const uint32_t KK = g.k * g.k, OHW = g.OH * g.OW, N = g.B * OHW, kdim = g.C * KK;
  using LA = DenseLoader<MT, false>;
  using LB = XPixLoader<128, CHUNK>;
  typename LA::Params pa{wA, kdim, g.OC, kdim, (kdim % 4 == 0) ? 1u : 0u};
  const uint32_t nch = CHUNK ? g.C / KT : 1;
  typename LB::Params pb{x, g.C, g.H, g.W, g.k, g.s, g.p, g.OW, OHW, N, kdim, nch,
                         make_fastdiv(OHW), make_fastdiv(g.OW), make_fastdiv(g.k),
                         make_fastdiv(KK), make_fastdiv(nch)};
  EpiConvFwd::Params pe{y, bias, g.OC, OHW, N, act, make_fastdiv(OHW)};
  const uint32_t ktiles = CHUNK ? KK * nch : cdiv(kdim, KT);
  return launch<MT, 128, LA, LB, EpiConvFwd>(pa, pb, pe, g.OC, N, ktiles, 1, "conv_forward");
}

bool conv_forward(const float* x, const float* w, const float* bias, float* y,
                  const ConvGeom& g, uint32_t act) {
  const uint32_t KK = g.k * g.k;
  const bool chunk = (g.C % KT == 0) && g.k > 1;
  const float* wA = w;
  if (chunk) {
    float* wp = workspace(size_t(g.OC) * g.C * KK);
    if (!wp) return false;
    uint32_t n = g.OC * g.C * KK;
    hipLaunchKernelGGL(k_permute_w, dim3(cdiv(n, 256)), dim3(256), 0, stream(), w, wp, g.OC, g.C,
                       KK, 0);
    if (!check_launch("permute_w")) return false;
    wA = wp;
  }
  const double fl = 2.0 * g.OC * g.C * KK * double(g.B) * g.OH * g.OW;
  ProfScope prof("conv_fwd", fl, 4.0 * (double(g.B) * g.C * g.H * g.W + double(g.B) * g.OC * g.OH * g.OW));
  const int MT = pick_tile(g.OC);
  if (MT == 128) return chunk ? conv_fwd_t<128, true>(x, wA, bias, y, g, act)
                              : conv_fwd_t<128, false>(x, wA, bias, y, g, act);
  return chunk ? conv_fwd_t<64, true>(x, wA, bias, y, g, act)
               : conv_fwd_t<64, false>(x, wA, bias, y, g, act);
}

// ------------------------------------------------------------- conv dW/db
template <int MT, int NT>
static bool conv_dw_t(const float* dy, const float* y, const float* x, float* part,
                      float* dbPart, const ConvGeom& g, uint32_t splits) {
  const uint32_t KK = g.k * g.k, OHW = g.OH * g.OW, N = g.C * KK;
  const uint32_t nchunk = cdiv(OHW, KT);
  using LA = GLoader<MT>;
  using LB = XColLoader<NT>;
  typename LA::Params pa{dy, y, dbPart, g.OC, OHW, nchunk, make_fastdiv(nchunk)};
  typename LB::Params pb{x, g.C, g.H, g.W, g.k, g.s, g.p, g.OW, OHW, nchunk, N,
                         make_fastdiv(g.OW), make_fastdiv(g.k), make_fastdiv(KK),
                         make_fastdiv(nchunk)};
  EpiRowMajor::Params pe{part, g.OC, N, N, g.OC * N};
  return launch<MT, NT, LA, LB, EpiRowMajor>(pa, pb, pe, g.OC, N, g.B * nchunk, splits,
                                             "conv_backward_filter");
}

bool conv_backward_filter(const float* dy, const float* y, const float* x, float* dw,
                          float* db, const ConvGeom& g) {
  const uint32_t KK = g.k * g.k, OHW = g.OH * g.OW, N = g.C * KK, M = g.OC;
  const int MT = pick_tile(M), NT = pick_tile(N);
  const uint32_t ktiles = g.B * cdiv(OHW, KT);
  const uint32_t tiles = cdiv(M, MT) * cdiv(N, NT);
  const uint32_t splits = pick_splits(tiles, ktiles, 16);
  const size_t pw = size_t(splits) * M * N, pb = size_t(splits) * M;
  float* ws = workspace(pw + pb);
  if (!ws) return false;
  float* part = ws;
  float* dbPart = db ? ws + pw : nullptr;
  bool ok;
  {
    const double fl = 2.0 * M * double(N) * double(g.B) * OHW;
    ProfScope prof("conv_dw", fl,
                   4.0 * (double(g.B) * g.OC * OHW * (y ? 2 : 1) + double(g.B) * g.C * g.H * g.W + double(M) * N));
    if (MT == 128 && NT == 128)
      ok = conv_dw_t<128, 128>(dy, y, x, part, dbPart, g, splits);
    else if (MT == 128)
      ok = conv_dw_t<128, 64>(dy, y, x, part, dbPart, g, splits);
    else if (NT == 128)
      ok = conv_dw_t<64, 128>(dy, y, x, part, dbPart, g, splits);
    else
      ok = conv_dw_t<64, 64>(dy, y, x, part, dbPart, g, splits);
  }
  if (ok && dw) ok = splitk_sum(part, dw, M * N, splits);
  if (ok && db) ok = splitk_sum(dbPart, db, M, splits);
  return ok;
}

// ------------------------------------------------------------------ conv dX
template <int MT, bool CHUNK, bool S1>
static bool conv_dx_t(const float* dy, const float* y, const float* wA, float* dx,
                      const ConvGeom& g) {
  const uint32_t KK = g.k * g.k, HW = g.H * g.W, N = g.B * HW, kdim = g.OC * KK;
  using LA = DenseLoader<MT, false>;
  using LB = GPixLoader<128, CHUNK, S1>;
  typename LA::Params pa{wA, kdim, g.C, kdim, (kdim % 4 == 0) ? 1u : 0u};
  const uint32_t noc = CHUNK ? g.OC / KT : 1;
  typename LB::Params pb{dy, y, g.OC, g.H, g.W, g.k, g.s, g.p, g.OH, g.OW, N, kdim, noc,
                         make_fastdiv(HW), make_fastdiv(g.W), make_fastdiv(g.k),
                         make_fastdiv(KK), make_fastdiv(noc)};
  EpiConvDx::Params pe{dx, g.C, HW, N, make_fastdiv(HW)};
  const uint32_t ktiles = CHUNK ? KK * noc : cdiv(kdim, KT);
  return launch<MT, 128, LA, LB, EpiConvDx>(pa, pb, pe, g.C, N, ktiles, 1,
                                            "conv_backward_input");
}

template <int MT>
static bool conv_dx_mt(const float* dy, const float* y, const float* wA, float* dx,
                       const ConvGeom& g, bool chunk) {
  if (g.s == 1)
    return chunk ? conv_dx_t<MT, true, true>(dy, y, wA, dx, g)
                 : conv_dx_t<MT, false, true>(dy, y, wA, dx, g);
  return chunk ? conv_dx_t<MT, true, false>(dy, y, wA, dx, g)
               : conv_dx_t<MT, false, false>(dy, y, wA, dx, g);
}

bool conv_backward_input(const float* dy, const float* y, const float* w, float* dx,
                         const ConvGeom& g) {
  const uint32_t KK = g.k * g.k;
  const bool chunk = (g.OC % KT == 0);
  float* wp = workspace(size_t(g.OC) * g.C * KK);
  if (!wp) return false;
  const uint32_t n = g.OC * g.C * KK;
  hipLaunchKernelGGL(k_permute_w, dim3(cdiv(n, 256)), dim3(256), 0, stream(), w, wp, g.OC, g.C,
                     KK, chunk ? 1 : 2);
  if (!check_launch("permute_w")) return false;
  const double fl = 2.0 * g.OC * g.C * KK * double(g.B) * g.OH * g.OW;
  ProfScope prof("conv_dx", fl,
                 4.0 * (double(g.B) * g.OC * g.OH * g.OW * (y ? 2 : 1) + double(g.B) * g.C * g.H * g.W));
  const int MT = pick_tile(g.C);
  return MT == 128 ? conv_dx_mt<128>(dy, y, wp, dx, g, chunk)
                   : conv_dx_mt<64>(dy, y, wp, dx, g, chunk);
}

}  // namespace dce
