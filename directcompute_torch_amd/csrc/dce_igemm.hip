// fp32 implicit GEMM on CDNA4 matrix cores (v_mfma_f32_16x16x4_f32) for the
// convolution forward, filter gradient (dW), input gradient (dX) and the
// flagged dense GEMM of MatMulAlloc.
//
//   C[m, n] = sum_k A[m, k] * B[n, k]
//
// Workgroup: 256 threads = 4 wave64 owning an MT x NT output tile: for MT in
// {64, 128} the waves sit 2x2, each with an (MT/2) x (NT/2) block of 16x16
// accumulators; for the narrow tiles MT in {16, 32} (few output channels)
// they sit 1x4, each with an MT x (NT/4) block, or (KT = 64) each wave takes
// the whole tile over its own 16-deep slice of every K tile.  K advances in
// tiles of KT (16, 32 or 64) through a double buffered LDS stage with one
// barrier per tile; the next tile's global loads are in flight while the
// current one is multiplied.
//
// Every global load is a (predicated) 16-byte load of four consecutive
// elements ("quad"), into registers or straight into LDS.  An operand is
// staged in LDS in one of two layouts:
//   ROWK  [row][k], quads along k  (row stride KT)       -> ds_read_b128
//   KROW  [k][row], quads along rows                     -> 4 x ds_read_b32
// Both feed the MFMA with the same k order: in MFMA s of a 16-wide k slice,
// lane l (r = l % 16, g = l / 16) supplies A[r][4g + s] and B[4g + s][r], so
// the four MFMAs together cover k 0..15 (the matrix unit sums over g).  ROWK
// rows are unpadded with their quads XOR-swizzled by row; KROW rows at least
// 64 wide are unpadded and swizzled by k where the loader allows it, the
// others padded by 4 floats (see Stage).  A wave with 2 or 4 fragments of a KROW operand
// interleaves them row by row, so that one ds_read_b64 / b128 per k serves
// all of them (Stage::frags_rif).
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
// hands back as its "im2col" handle.  Two layer kinds take other operands:
// pointwise (1x1, stride 1) layers multiply the NCHW planes in place, and
// layers with fewer than 4 input channels read a stride-phase copy of x
// (stride-phase section below).
// Split-K writes partial tiles (split z is the slowest index of the tile
// numbering) that a second pass sums in a fixed order; nothing uses atomics,
// so results are deterministic.
#include "dce_internal.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <type_traits>

namespace dce {

constexpr int kThreads = 256;
static inline uint32_t cdiv(uint64_t a, uint64_t b) { return uint32_t((a + b - 1) / b); }

// ---------------------------------------------------------------------------
// LDS stage geometry of one operand.
// ---------------------------------------------------------------------------
template <int R, int KT, bool KROW, bool SWZOK = true>
struct Stage {
  // ROWK rows are KT floats, unpadded.  Measured with an LDS probe on gfx950
  // (64 banks): 16-byte stores of the loaders' ROWK pattern (KQ quads of
  // consecutive rows) run 15% slower with a +4 pad than without, while the
  // fragment reads (one quad of 16 consecutive rows) cost the same either way.
  // KROW rows of at least 64 floats (SWZ, when the loader opts in) are
  // unpadded too, with the row-quad index XOR-swizzled by k (fk): a fragment
  // read takes one float of 16 consecutive rows at 4 k's 4 apart, which the
  // swizzle spreads over all 64 banks (unswizzled, k rows R floats apart
  // would share banks).  Other KROW rows keep a +4 pad.  Unpadded stages take
  // direct global-to-LDS loads, the conv dW operands included (the G rows
  // and the per-quad tap rows of x: AlexNet's conv backward 112.3 -> 113.0
  // -> 113.7 TFLOP/s as each went direct).
  static constexpr bool SWZ = KROW && SWZOK && R >= 64;
  static constexpr int LD = KROW ? (SWZ ? R : R + 4) : KT;
  static constexpr int SIZE = KROW ? KT * LD : R * LD;
  static constexpr int KQ = KT / 4;
  static constexpr int RQ = R / 4;
  // NQ quads per stage.  A narrow operand (NQ < kThreads) is staged by the
  // first NQ threads, one quad each; the others load and store nothing.
  static constexpr int NQ = R * KT / 4;
  static_assert(NQ % kThreads == 0 || kThreads % NQ == 0, "tile must split evenly over the workgroup");
  static constexpr bool PART = NQ < kThreads;
  static constexpr int Q = PART ? 1 : NQ / kThreads;
  __device__ static __forceinline__ bool active(int t) { return !PART || t < NQ; }
  // Quad i of thread t.  ROWK: consecutive lanes take consecutive k-quads of
  // one row; KROW: consecutive lanes take consecutive row-quads of one k.
  // kThreads is a multiple of KQ and RQ, so quad i sits DROW rows (ROWK) or
  // DK k-steps (KROW) past quad 0, and DLDS floats past it in LDS.
  static constexpr int DROW = KROW ? 0 : kThreads / KQ;
  static constexpr int DK = KROW ? kThreads / RQ : 0;
  static constexpr int DLDS = KROW ? DK * LD : DROW * LD;
  // ROWK quad swizzle: logical k-quad q of row `row` sits at physical quad
  // q ^ fr(row).  A fragment read takes quad q of 16 consecutive rows; rows
  // are KT floats, so 64 / KT consecutive rows fill the 64 banks once and the
  // unswizzled quads of rows 64 / KT apart share banks (4-way conflicts at
  // KT = 16, 16-way at KT = 64).  fr spreads the 16 rows over all 64 banks.
  // Thread t still owns the 16-byte slot t of its row group (the direct
  // loads' lane order); it loads the logical quad that belongs there.
  static_assert(KROW || (KT <= 64 && 64 % KT == 0), "ROWK swizzle period");
  static_assert(KROW || Q == 1 || DROW % 16 == 0, "fr is periodic in 16 rows");
  __device__ static __forceinline__ int fr(int row) { return (row / (64 / KT)) % KQ; }
  __device__ static __forceinline__ int qrow(int t, int i) {
    return KROW ? 4 * (t % RQ) : t / KQ + DROW * i;
  }
  // Logical k offset of the data in thread t's quad i (DROW is a multiple of
  // fr's 16-row period, so it is the same for every i).
  __device__ static __forceinline__ int qk(int t, int i) {
    return KROW ? t / RQ + DK * i : 4 * ((t % KQ) ^ fr(t / KQ));
  }
  __device__ static __forceinline__ int lds_off(int t) {
    return KROW ? qk(t, 0) * LD + qrow(t, 0) : qrow(t, 0) * LD + 4 * (t % KQ);
  }
  // SWZ: logical row quad rq of k row k sits at physical quad rq ^ fk(k).
  __device__ static __forceinline__ int fk(int k) { return 4 * ((k >> 2) & 3); }
  // The logical first row of quad i of thread t (its physical slot is
  // lds_off(t) + i * DLDS): KROW rows are swizzled back from the slot.
  __device__ static __forceinline__ int qrow_data(int t, int i) {
    if (!SWZ) return qrow(t, i);
    return 4 * ((t % RQ) ^ fk(qk(t, i)));
  }
  static constexpr bool kRow = KROW;
  // KROW, F = 2 or 4 fragments read together ("row-interleaved"): fragment i
  // takes rows rb + F*rho + i (rho = 0..15), so lane (r, g) finds the F
  // fragments' values at k = kb + 4g + s in F consecutive floats of one k row
  // (inside one row quad, so the SWZ swizzle moves them together): one
  // ds_read_b64 / b128 per s instead of F ds_read_b32.  The epilogues map the
  // accumulator rows back (frow).
  template <int F>
  __device__ static __forceinline__ void frags_rif(const float* S, int rb, int r, int g, int kb,
                                                   f4 (&out)[F]) {
    static_assert(KROW && (F == 2 || F == 4), "row-interleaved fragments: KROW, F in {2, 4}");
    const int row = rb + F * r;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int k = kb + 4 * g + s;
      const float* p = S + k * LD + (SWZ ? 4 * ((row >> 2) ^ fk(k)) + (row & 3) : row);
      if constexpr (F == 4) {
        const f4 v = *reinterpret_cast<const f4*>(p);
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i][s] = v[i];
      } else {
        const f2 v = *reinterpret_cast<const f2*>(p);
        out[0][s] = v[0];
        out[1][s] = v[1];
      }
    }
  }
  // MFMA operand of 16 rows starting at rb, k slice kb: components s = 0..3.
  __device__ static __forceinline__ f4 frag(const float* S, int rb, int r, int g, int kb) {
    if (!KROW) return *reinterpret_cast<const f4*>(S + (rb + r) * LD + 4 * ((kb / 4 + g) ^ fr(rb + r)));
    f4 v;
    const int row = rb + r;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int k = kb + 4 * g + s;
      v[s] = SWZ ? S[k * LD + 4 * ((row >> 2) ^ fk(k)) + (row & 3)] : S[k * LD + row];
    }
    return v;
  }
};

template <class St>
struct LoaderBase {
  static constexpr int Q = St::Q;
  // LDSD: the operand goes global -> LDS directly (buffer_load ... lds).  Only
  // the unpadded [row][k] stages qualify: there a wave's 64 quads of one load
  // are 64 consecutive 16-byte LDS slots in lane order (lds_off(t) = 4 t).
  static constexpr bool LDSD = false;
  // As the B operand: accumulate C transposed (MFMA B fragment first).
  static constexpr bool kTransAcc = false;
  int lds0, wbase;
  bool act;
  __device__ __forceinline__ void base_init(int tid) {
    lds0 = St::lds_off(tid);
    // Wave-uniform, so M0 of the direct loads is set with scalar arithmetic.
    wbase = __builtin_amdgcn_readfirstlane(St::lds_off(tid & ~63));
    act = St::active(tid);
  }
  __device__ __forceinline__ void store(float* S, const f4 (&r)[Q]) const {
    if (St::PART && !act) return;
#pragma unroll
    for (int i = 0; i < Q; ++i) *reinterpret_cast<f4*>(S + lds0 + i * St::DLDS) = r[i];
  }
};

__device__ __forceinline__ f4 zero4() { return f4{0.f, 0.f, 0.f, 0.f}; }

// ---------------------------------------------------------------------------
// Dense operands.  Preconditions (the host pads copies to meet them): 16-byte
// aligned base, ld % 4 == 0, and kdim (ROWK) / rows (KROW) a multiple of 4, so
// a quad is either wholly inside the matrix or wholly padding.
// ---------------------------------------------------------------------------
// [rows][kdim] row-major (ROWK).
template <int R, int KT>
struct LdDenseRK : LoaderBase<Stage<R, KT, false>> {
  using St = Stage<R, KT, false>;
  static constexpr bool KROW = false;
  using LoaderBase<St>::Q;
  struct Params {
    const float* p;
    uint32_t ld, rows, kdim, n;  // n: floats in the buffer
  };
  BRes b;
  uint32_t kdim, kq;
  uint32_t base[Q];
  __device__ __forceinline__ void init(const Params& P, uint32_t row0, int tid) {
    this->base_init(tid);
    b.init(P.p, P.n);
    kdim = P.kdim;
    kq = St::qk(tid, 0);
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t row = row0 + St::qrow(tid, i);
      base[i] = (this->act && row < P.rows) ? row * P.ld + kq : kOob;
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
    const uint32_t k0 = kt * KT;
    const bool kok = k0 + kq < kdim;
#pragma unroll
    for (int i = 0; i < Q; ++i) r[i] = b.ld4(kok ? base[i] + k0 : kOob);
  }
  static constexpr bool LDSD = true;
  __device__ __forceinline__ void issue_lds(uint32_t kt, float* S) const {
    if (St::PART && !this->act) return;  // whole waves (NQ is a multiple of 64)
    const uint32_t k0 = kt * KT;
    const bool kok = k0 + kq < kdim;
#pragma unroll
    for (int i = 0; i < Q; ++i) b.ld4_lds(kok ? base[i] + k0 : kOob, S + this->wbase + i * St::DLDS);
  }
};

// [kdim][rows] k-major (KROW).
template <int R, int KT>
struct LdDenseKR : LoaderBase<Stage<R, KT, true>> {
  using St = Stage<R, KT, true>;
  static constexpr bool KROW = true;
  using LoaderBase<St>::Q;
  struct Params {
    const float* p;
    uint32_t ld, rows, kdim, n;
  };
  BRes b;
  uint32_t kdim, ld, kk0;
  uint32_t base[Q];  // quad i's offset at k tile 0, or kOob for rows past the matrix
  __device__ __forceinline__ void init(const Params& P, uint32_t row0, int tid) {
    this->base_init(tid);
    b.init(P.p, P.n);
    kdim = P.kdim;
    ld = P.ld;
    kk0 = St::qk(tid, 0);
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t row = row0 + St::qrow_data(tid, i);
      base[i] = (this->act && row < P.rows) ? (kk0 + St::DK * i) * P.ld + row : kOob;
    }
  }
  __device__ __forceinline__ void offsets(uint32_t kt, uint32_t (&o)[Q]) const {
    const uint32_t k0 = kt * KT;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t k = k0 + kk0 + St::DK * i;
      o[i] = k < kdim ? base[i] + k0 * ld : kOob;
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
    uint32_t o[Q];
    offsets(kt, o);
#pragma unroll
    for (int i = 0; i < Q; ++i) r[i] = b.ld4(o[i]);
  }
  static constexpr bool LDSD = St::SWZ;
  __device__ __forceinline__ void issue_lds(uint32_t kt, float* S) const {
    uint32_t o[Q];
    offsets(kt, o);
#pragma unroll
    for (int i = 0; i < Q; ++i) b.ld4_lds(o[i], S + this->wbase + i * St::DLDS);
  }
};

// ---------------------------------------------------------------------------
// NCHW operands of the pointwise (1 x 1, stride 1, no padding) convolutions,
// read in place: a pixel n = b*HW + pix of channel ch is src[(b*Ch + ch)*HW
// + pix].  HW % 4 == 0, so four consecutive pixels (a quad) lie in one image.
// ---------------------------------------------------------------------------
// KROW: rows = pixels n, k = channel (zero for k >= Ch or n >= N).
struct NchwKRParams {
  const float* src;
  uint32_t Ch, HW, N, n;
  FastDiv dHW;
};
template <int R, int KT>
struct LdNchwKR : LoaderBase<Stage<R, KT, true>> {
  using St = Stage<R, KT, true>;
  static constexpr bool KROW = true;
  static constexpr bool kTransAcc = true;  // pixel columns: quad stores
  using LoaderBase<St>::Q;
  using Params = NchwKRParams;
  BRes b;
  uint32_t Ch, HW, kk0;
  uint32_t base[Q];  // quad i's offset at channel 0, or kOob past the pixels
  __device__ __forceinline__ void init(const Params& P, uint32_t row0, int tid) {
    this->base_init(tid);
    b.init(P.src, P.n);
    Ch = P.Ch;
    HW = P.HW;
    kk0 = St::qk(tid, 0);
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t n = row0 + St::qrow_data(tid, i);
      const uint32_t bb = fdiv(n, P.dHW);
      base[i] = (this->act && n < P.N) ? bb * P.Ch * P.HW + (n - bb * P.HW) : kOob;
    }
  }
  __device__ __forceinline__ void offsets(uint32_t kt, uint32_t (&o)[Q]) const {
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t ch = kt * KT + kk0 + St::DK * i;
      o[i] = (base[i] != kOob && ch < Ch) ? base[i] + ch * HW : kOob;
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
    uint32_t o[Q];
    offsets(kt, o);
#pragma unroll
    for (int i = 0; i < Q; ++i) r[i] = b.ld4(o[i]);
  }
  static constexpr bool LDSD = St::SWZ;
  __device__ __forceinline__ void issue_lds(uint32_t kt, float* S) const {
    uint32_t o[Q];
    offsets(kt, o);
#pragma unroll
    for (int i = 0; i < Q; ++i) b.ld4_lds(o[i], S + this->wbase + i * St::DLDS);
  }
};

// ROWK: rows = channels, k = pixel n over the batch (the pointwise dW
// operands).  Row `onesRow` (when below R rows of the grid) reads 1 for
// every k < K, from a 4-float buffer of ones: the dW GEMM then yields the
// bias gradient, sum over k of the other operand, as its extra column.
struct NchwRKParams {
  const float* src;
  const float* ones;
  uint32_t Ch, HW, K, n, onesRow;
  FastDiv dHW;
};
template <int R, int KT>
struct LdNchwRK : LoaderBase<Stage<R, KT, false>> {
  using St = Stage<R, KT, false>;
  static constexpr bool KROW = false;
  using LoaderBase<St>::Q;
  using Params = NchwRKParams;
  BRes b, bo;
  uint32_t Ch, HW, K, kq;
  FastDiv dHW;
  uint32_t rowoff[Q];  // quad i's channel offset ch * HW, or kOob past the channels
  bool one[Q];
  __device__ __forceinline__ void init(const Params& P, uint32_t row0, int tid) {
    this->base_init(tid);
    b.init(P.src, P.n);
    bo.init(P.ones, 4);
    Ch = P.Ch;
    HW = P.HW;
    K = P.K;
    dHW = P.dHW;
    kq = St::qk(tid, 0);
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t r = row0 + St::qrow(tid, i);
      one[i] = this->act && r == P.onesRow;
      rowoff[i] = (this->act && r < P.Ch) ? r * P.HW : kOob;
    }
  }
  // The thread's quads share their k (ROWK): one image / pixel split per tile.
  __device__ __forceinline__ void offsets(uint32_t kt, uint32_t (&o)[Q]) const {
    const uint32_t k0 = kt * KT + kq;
    const uint32_t bb = fdiv(k0, dHW);
    const uint32_t img = bb * Ch * HW + (k0 - bb * HW);
#pragma unroll
    for (int i = 0; i < Q; ++i) o[i] = (rowoff[i] != kOob && k0 < K) ? img + rowoff[i] : kOob;
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
    uint32_t o[Q];
    offsets(kt, o);
    const bool kin = kt * KT + kq < K;
#pragma unroll
    for (int i = 0; i < Q; ++i) r[i] = one[i] ? bo.ld4(kin ? 0u : kOob) : b.ld4(o[i]);
  }
  static constexpr bool LDSD = true;
  __device__ __forceinline__ void issue_lds(uint32_t kt, float* S) const {
    if (St::PART && !this->act) return;  // whole waves (NQ is a multiple of 64)
    uint32_t o[Q];
    offsets(kt, o);
    const bool kin = kt * KT + kq < K;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      float* dst = S + this->wbase + i * St::DLDS;
      if (one[i])
        bo.ld4_lds(kin ? 0u : kOob, dst);
      else
        b.ld4_lds(o[i], dst);
    }
  }
};

// ---------------------------------------------------------------------------
// Pixel-row gather over an NHWC source (ROWK): rows = pixels of a grid
// (b, a, c); k runs over the taps (kh, kw) and the Cp source channels (Cp the
// padded channel count, Cp % 4 == 0) in one of two orders:
//   flat    (BLK false): k = (kh * k + kw) * Cp + ch;
//   blocked (BLK true, Cp % kCB == 0, KT == kCB):
//           k = (cb * KK + kh * k + kw) * kCB + ci, ch = cb * kCB + ci.
// The blocked order makes a K tile one tap of one channel block, so a block's
// slice of the source stays in L1 while all KK taps walk over it (the flat
// order re-fetches each source pixel once per tap when Cp is large).  Within
// a thread, all quads share their k (ROWK), so the tap decomposition is done
// once per K tile.
//   FWD: source = x, rows = output pixels, tap reads x[b, a*s + kh - p, c*s + kw - p].
//   !FWD (dX): source = G, rows = input pixels, tap reads G[b, oh, ow] with
//        oh*s == a + p - kh exactly (S1: s == 1, no divisibility test).
//        A strided dX runs as s*s sub-pixel phases, each an S1 gather over
//        its own grid of input pixels with nh x nw taps (k = nw) and the
//        column origin shifted by pwd (phase_dx below).
// ---------------------------------------------------------------------------
constexpr int kCB = 16;

template <int R, int KT, bool FWD, bool S1, bool BLK>
struct LdPixRK : LoaderBase<Stage<R, KT, false>> {
  static_assert(!BLK || KT == kCB, "blocked order: one K tile per (channel block, tap)");
  static_assert(!Stage<R, KT, false>::PART, "pixel operands fill the workgroup");
  using St = Stage<R, KT, false>;
  static constexpr bool KROW = false;
  using LoaderBase<St>::Q;
  struct Params {
    const float* src;
    uint32_t srcH, srcW, Cp, k, s, p;
    uint32_t gridW, gridHW, N, kdim, n;
    FastDiv dGridHW, dGridW, dInner, dK;  // dInner: KK (blocked) or Cp (flat)
    int pwd;  // dX: the column origin is c + p + pwd (0 but for the sub-pixel phases)
  };
  // FAST (blocked order, forward or stride-1 dX): the K tile's tap and
  // channel block are wave-uniform, so a quad's source offset is a per-quad
  // constant qbase plus a uniform tap term -- no per-tile multiplies.
  static constexpr bool FAST = BLK && (FWD || S1);
  static constexpr bool kTransAcc = true;  // pixel columns: quad stores (measured faster)
  BRes b;
  uint32_t srcH, srcW, Cp, k, s, kdim, kq;
  FastDiv dInner, dK;
  uint32_t pbase[Q], qbase[Q];
  int r0[Q], c0[Q];
  __device__ __forceinline__ void init(const Params& P, uint32_t row0, int tid) {
    this->base_init(tid);
    b.init(P.src, P.n);
    srcH = P.srcH;
    srcW = P.srcW;
    Cp = P.Cp;
    k = P.k;
    s = P.s;
    kdim = P.kdim;
    dInner = P.dInner;
    dK = P.dK;
    kq = St::qk(tid, 0);
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t n = row0 + St::qrow(tid, i);
      const uint32_t bb = fdiv(n, P.dGridHW);
      const uint32_t rem = n - bb * P.gridHW;
      const uint32_t a = fdiv(rem, P.dGridW);
      const uint32_t c = rem - a * P.gridW;
      pbase[i] = bb * P.srcH * P.srcW;
      if (FWD) {
        r0[i] = int(a * P.s) - int(P.p);
        c0[i] = int(c * P.s) - int(P.p);
      } else {
        r0[i] = int(a + P.p);
        c0[i] = int(c + P.p) + P.pwd;
      }
      // A row past the grid gets an origin no tap can bring into the image.
      if (n >= P.N) r0[i] = FWD ? -(1 << 20) : (1 << 20);
      // Offset of tap (0, 0), channel kq, modulo 2^32 (the origin may lie
      // in the padding); only in-image taps are ever used.
      qbase[i] = (pbase[i] + uint32_t(r0[i]) * P.srcW + uint32_t(c0[i])) * P.Cp + kq;
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
    uint32_t off[Q];
    offsets(kt, off);
#pragma unroll
    for (int i = 0; i < Q; ++i) r[i] = b.ld4(off[i]);
  }
  static constexpr bool LDSD = true;
  __device__ __forceinline__ void issue_lds(uint32_t kt, float* S) const {
    uint32_t off[Q];
    offsets(kt, off);
#pragma unroll
    for (int i = 0; i < Q; ++i) b.ld4_lds(off[i], S + this->wbase + i * St::DLDS);
  }
  __device__ __forceinline__ void offsets(uint32_t kt, uint32_t (&o)[Q]) const {
    if constexpr (FAST) {
      const uint32_t cb = fdiv(kt, dInner);
      const uint32_t khw = kt - cb * dInner.d;
      const uint32_t kh = fdiv(khw, dK);
      const uint32_t kw = khw - kh * k;
      const bool kok = cb * kCB < Cp;  // Cp % kCB == 0: the whole tile or none
      const uint32_t tap = (kh * srcW + kw) * Cp;
      const uint32_t toff = FWD ? cb * kCB + tap : cb * kCB - tap;
#pragma unroll
      for (int i = 0; i < Q; ++i) {
        const int h = FWD ? r0[i] + int(kh) : r0[i] - int(kh);
        const int w = FWD ? c0[i] + int(kw) : c0[i] - int(kw);
        const bool ok = kok && uint32_t(h) < srcH && uint32_t(w) < srcW;
        o[i] = ok ? qbase[i] + toff : kOob;
      }
      return;
    }
    uint32_t khw, ch;
    bool kok;
    if (BLK) {
      const uint32_t cb = fdiv(kt, dInner);
      khw = kt - cb * dInner.d;
      ch = cb * kCB + kq;
      kok = ch < Cp;
    } else {
      const uint32_t kk0 = kt * KT + kq;
      khw = fdiv(kk0, dInner);
      ch = kk0 - khw * Cp;
      kok = kk0 < kdim;
    }
    const uint32_t kh = fdiv(khw, dK);
    const uint32_t kw = khw - kh * k;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      int h, w;
      bool ok = kok;
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
      o[i] = ok ? (pbase[i] + uint32_t(h) * srcW + uint32_t(w)) * Cp + ch : kOob;
    }
  }
};

// ---------------------------------------------------------------------------
// dW operands (KROW, k = flat output pixel over the batch).
// ---------------------------------------------------------------------------
// A: G rows oc, element (oc, pix) = G_nhwc[pix*OCp + oc].
struct GradKRParams {
  const float* g;
  uint32_t OCp, npix, n;
};
template <int R, int KT>
struct LdGradKR : LoaderBase<Stage<R, KT, true>> {
  using St = Stage<R, KT, true>;
  static constexpr bool KROW = true;
  using LoaderBase<St>::Q;
  using Params = GradKRParams;
  BRes b;
  uint32_t OCp, npix, kk0;
  uint32_t base[Q];  // quad i's offset at k tile 0, or kOob for channels past OCp
  __device__ __forceinline__ void init(const Params& P, uint32_t row0, int tid) {
    this->base_init(tid);
    b.init(P.g, P.n);
    OCp = P.OCp;
    npix = P.npix;
    kk0 = St::qk(tid, 0);
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t oc = row0 + St::qrow_data(tid, i);
      base[i] = (this->act && oc < P.OCp) ? (kk0 + St::DK * i) * P.OCp + oc : kOob;
    }
  }
  __device__ __forceinline__ void offsets(uint32_t kt, uint32_t (&o)[Q]) const {
    const uint32_t p0 = kt * KT;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t pix = p0 + kk0 + St::DK * i;
      o[i] = pix < npix ? base[i] + p0 * OCp : kOob;
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
    uint32_t o[Q];
    offsets(kt, o);
#pragma unroll
    for (int i = 0; i < Q; ++i) r[i] = b.ld4(o[i]);
  }
  static constexpr bool LDSD = St::SWZ;
  __device__ __forceinline__ void issue_lds(uint32_t kt, float* S) const {
    uint32_t o[Q];
    offsets(kt, o);
#pragma unroll
    for (int i = 0; i < Q; ++i) b.ld4_lds(o[i], S + this->wbase + i * St::DLDS);
  }
};

// B: x taps, rows n = (kh, kw, c) (c fastest, Cp), element (n, pix) =
// x_nhwc[b, oh*s + kh - p, ow*s + kw - p, c] or 0 outside the image.
struct XTapParams {
  const float* x;
  uint32_t H, W, Cp, k, s, p, OW, OHW, npix, N, n;
  FastDiv dOHW, dOW, dCp, dK;
};
template <int R, int KT>
struct LdXTapKR : LoaderBase<Stage<R, KT, true>> {
  using St = Stage<R, KT, true>;
  static constexpr bool KROW = true;
  using LoaderBase<St>::Q;
  using Params = XTapParams;
  BRes b;
  uint32_t H, W, Cp, s, OW, OHW, npix, kk0;
  FastDiv dOHW, dOW;
  // Quad i's tap row: channel offset and tap origin (kh, kw); with the
  // swizzled stage the quads of one thread sit on different tap rows.
  uint32_t off[Q];
  int kh[Q], kw[Q];
  __device__ __forceinline__ void init(const Params& P, uint32_t row0, int tid) {
    this->base_init(tid);
    b.init(P.x, P.n);
    H = P.H;
    W = P.W;
    Cp = P.Cp;
    s = P.s;
    OW = P.OW;
    OHW = P.OHW;
    npix = P.npix;
    dOHW = P.dOHW;
    dOW = P.dOW;
    kk0 = St::qk(tid, 0);
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t n = row0 + St::qrow_data(tid, i);
      const uint32_t khw = fdiv(n, P.dCp);
      off[i] = n - khw * P.Cp;
      const uint32_t a = fdiv(khw, P.dK);
      kh[i] = int(a) - int(P.p);
      kw[i] = int(khw - a * P.k) - int(P.p);
      // A row past the taps (or a thread that stages nothing) gets an offset
      // no pixel can bring into the image.
      if (n >= P.N || !this->act) kh[i] = -(1 << 20);
    }
  }
  __device__ __forceinline__ void offsets(uint32_t kt, uint32_t (&o)[Q]) const {
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t pix = kt * KT + kk0 + St::DK * i;
      const uint32_t bb = fdiv(pix, dOHW);
      const uint32_t rem = pix - bb * OHW;
      const uint32_t oh = fdiv(rem, dOW);
      const uint32_t ow = rem - oh * OW;
      const int ih = int(oh * s) + kh[i];
      const int iw = int(ow * s) + kw[i];
      const bool ok = pix < npix && uint32_t(ih) < H && uint32_t(iw) < W;
      o[i] = ok ? ((bb * H + uint32_t(ih)) * W + uint32_t(iw)) * Cp + off[i] : kOob;
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
    uint32_t o[Q];
    offsets(kt, o);
#pragma unroll
    for (int i = 0; i < Q; ++i) r[i] = b.ld4(o[i]);
  }
  static constexpr bool LDSD = St::SWZ;
  __device__ __forceinline__ void issue_lds(uint32_t kt, float* S) const {
    uint32_t o[Q];
    offsets(kt, o);
#pragma unroll
    for (int i = 0; i < Q; ++i) b.ld4_lds(o[i], S + this->wbase + i * St::DLDS);
  }
};

// ---------------------------------------------------------------------------
// Channel-packed source for convolutions over C < 4 channels: x copied by
// k_to_pk to [B][Hp][Wp][C] (Hp = H + 2p, Wp = W + 2p, zero border), and the
// unpadded tap order t = kh * kC + j with kC = k * C, j = kw * C + c (kdim =
// k * kC; the NHWC layout would pad C to 4 and waste up to 3/4 of the
// tap axis).  For every output pixel a kernel row's kC values are contiguous,
// so a quad of 4 consecutive t is one 16-byte load (4-byte aligned) unless it
// runs past the end of its kernel row (j + 3 >= kC): its tail then comes from
// a second load at the next kernel row, shifted so that element e lines up
// (from t's row origin + rowp - (kC - j)).  Tail elements past the last
// kernel row read as zeros.
// ---------------------------------------------------------------------------
struct PkParams {
  const float* src;
  uint32_t rowp, imgp, C, k, s, kC, kdim;  // rowp = Wp * C, imgp = Hp * Wp * C
  uint32_t OW, OHW, npix, n;               // n: floats in the copy
  FastDiv dOHW, dOW, dKC;
};

// Offset of output pixel pix's window origin in the packed copy.
__device__ __forceinline__ uint32_t pk_origin(const PkParams& P, uint32_t pix) {
  const uint32_t bb = fdiv(pix, P.dOHW);
  const uint32_t rem = pix - bb * P.OHW;
  const uint32_t oh = fdiv(rem, P.dOW);
  const uint32_t ow = rem - oh * P.OW;
  return bb * P.imgp + oh * P.s * P.rowp + ow * P.s * P.C;
}

// Quad of taps t..t+3 at a window origin: o1 = t's offset from the origin,
// o2 = the shifted next-row offset (kOob: none), m = elements left in t's row.
__device__ __forceinline__ f4 pk_quad(const BRes& b, bool ok, uint32_t org, uint32_t o1,
                                      uint32_t o2, uint32_t m) {
  f4 v = b.ld4(ok && o1 != kOob ? org + o1 : kOob);
  if (m < 4) {
    const f4 w = b.ld4(ok && o2 != kOob ? org + o2 : kOob);
#pragma unroll
    for (int e = 1; e < 4; ++e)
      if (uint32_t(e) >= m) v[e] = w[e];
  }
  return v;
}

// Row-origin offsets of tap t (shared by the two loaders below).
__device__ __forceinline__ void pk_tap(const PkParams& P, uint32_t t, uint32_t& o1, uint32_t& o2,
                                       uint32_t& m) {
  if (t >= P.kdim) {
    o1 = o2 = kOob;
    m = 4;
    return;
  }
  const uint32_t kh = fdiv(t, P.dKC), j = t - kh * P.kC;
  m = P.kC - j;
  o1 = kh * P.rowp + j;
  o2 = (m < 4 && kh + 1 < P.k) ? (kh + 1) * P.rowp - m : kOob;
}

// Forward B operand (ROWK): rows = output pixels, k = packed taps.  All quads
// of a thread share their taps, so the tap split is done once per K tile.
template <int R, int KT>
struct LdPkRK : LoaderBase<Stage<R, KT, false>> {
  static_assert(!Stage<R, KT, false>::PART, "pixel operands fill the workgroup");
  using St = Stage<R, KT, false>;
  static constexpr bool KROW = false;
  using LoaderBase<St>::Q;
  using Params = PkParams;
  BRes b;
  PkParams P;
  uint32_t kq;
  uint32_t org[Q];
  bool ok[Q];
  __device__ __forceinline__ void init(const Params& p, uint32_t row0, int tid) {
    this->base_init(tid);
    P = p;
    b.init(p.src, p.n);
    kq = St::qk(tid, 0);
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t pix = row0 + St::qrow(tid, i);
      ok[i] = pix < p.npix;
      org[i] = ok[i] ? pk_origin(p, pix) : 0u;
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
    uint32_t o1, o2, m;
    pk_tap(P, kt * KT + kq, o1, o2, m);
#pragma unroll
    for (int i = 0; i < Q; ++i) r[i] = pk_quad(b, ok[i], org[i], o1, o2, m);
  }
};

// dW operand (KROW): rows = packed taps, k = output pixels.  A thread's quads
// keep their taps for the whole K loop; the pixel walks.
template <int R, int KT>
struct LdPkKR : LoaderBase<Stage<R, KT, true, false>> {
  using St = Stage<R, KT, true, false>;
  static constexpr bool KROW = true;
  using LoaderBase<St>::Q;
  using Params = PkParams;
  BRes b;
  PkParams P;
  uint32_t kk0;
  uint32_t o1[Q], o2[Q], m[Q];
  __device__ __forceinline__ void init(const Params& p, uint32_t row0, int tid) {
    this->base_init(tid);
    P = p;
    b.init(p.src, p.n);
    kk0 = St::qk(tid, 0);
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      pk_tap(p, this->act ? row0 + St::qrow_data(tid, i) : p.kdim, o1[i], o2[i], m[i]);
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t pix = kt * KT + kk0 + St::DK * i;
      const bool ok = pix < P.npix;
      r[i] = pk_quad(b, ok, ok ? pk_origin(P, pix) : 0u, o1[i], o2[i], m[i]);
    }
  }
};

// ---------------------------------------------------------------------------
// Stride-phase copy for convolutions over C < 4 channels with stride S <= 4
// (k_to_ps): xs[((b*Hp + r)*C + c)*S + ph][col] = x[b][c][r - p][col*S + ph
// - p] (zero outside the image), rows of Ncol floats (Ncol % 4 == 0), Hp =
// H + 2p.  The output pixels form a padded grid (b, oh, ow) with ow < OWp =
// pad4(OW); the extra columns are computed and dropped (their G is zero).
// Tap t = (c*k + kh)*k + kw of output pixel (b, oh, ow) reads
//   xs[pixel part (b*Hp + oh*S)*RS + ow] + [tap part (kh*C + c)*S*Ncol +
//   (kw % S)*Ncol + kw / S],  RS = C*S*Ncol,
// so four consecutive output pixels of one tap are four consecutive floats:
// a quad never straddles anything (taps or pixels), unlike the channel-packed
// layout whose tap quads straddle kernel rows.  Quads start at 4-byte
// alignment (kw / S); the GPU runs with unaligned access enabled.
// ---------------------------------------------------------------------------
struct PsParams {
  const float* src;
  uint32_t RS, Hp, S, Ncol, C, k, KK, kdim;  // kdim = C*KK taps
  uint32_t OWp, OHWp, npix, n;               // npix = B*OHWp padded pixels; n: floats
  FastDiv dOHWp, dOWp, dKK, dK, dS;
};

__device__ __forceinline__ uint32_t ps_pixel(const PsParams& P, uint32_t n) {
  const uint32_t b = fdiv(n, P.dOHWp), rem = n - b * P.OHWp;
  const uint32_t oh = fdiv(rem, P.dOWp), ow = rem - oh * P.OWp;
  return (b * P.Hp + oh * P.S) * P.RS + ow;
}
__device__ __forceinline__ uint32_t ps_tap(const PsParams& P, uint32_t t) {
  const uint32_t c = fdiv(t, P.dKK), r = t - c * P.KK;
  const uint32_t kh = fdiv(r, P.dK), kw = r - kh * P.k;
  const uint32_t cq = fdiv(kw, P.dS), ph = kw - cq * P.S;
  return ((kh * P.C + c) * P.S + ph) * P.Ncol + cq;
}

// Forward B operand (KROW): rows = padded output pixels, k = taps.  A
// thread's quads share one row quad (4 pixels, fixed for the K loop).
template <int R, int KT>
struct LdPsKR : LoaderBase<Stage<R, KT, true, false>> {
  using St = Stage<R, KT, true, false>;
  static constexpr bool KROW = true;
  static constexpr bool kTransAcc = true;  // pixel columns: quad stores (measured faster)
  using LoaderBase<St>::Q;
  using Params = PsParams;
  BRes b;
  PsParams P;
  uint32_t kk0, pbase;
  __device__ __forceinline__ void init(const Params& p, uint32_t row0, int tid) {
    this->base_init(tid);
    P = p;
    b.init(p.src, p.n);
    kk0 = St::qk(tid, 0);
    const uint32_t n0 = row0 + St::qrow_data(tid, 0);
    pbase = (this->act && n0 < p.npix) ? ps_pixel(p, n0) : kOob;
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t t = kt * KT + kk0 + St::DK * i;
      r[i] = b.ld4(pbase != kOob && t < P.kdim ? pbase + ps_tap(P, t) : kOob);
    }
  }
};

// dW operand (ROWK): rows = taps (fixed per thread), k = padded pixels.
template <int R, int KT>
struct LdPsRK : LoaderBase<Stage<R, KT, false>> {
  using St = Stage<R, KT, false>;
  static constexpr bool KROW = false;
  using LoaderBase<St>::Q;
  using Params = PsParams;
  BRes b;
  PsParams P;
  uint32_t kq;
  uint32_t toff[Q];
  __device__ __forceinline__ void init(const Params& p, uint32_t row0, int tid) {
    this->base_init(tid);
    P = p;
    b.init(p.src, p.n);
    kq = St::qk(tid, 0);
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t t = row0 + St::qrow(tid, i);
      toff[i] = (this->act && t < p.kdim) ? ps_tap(p, t) : kOob;
    }
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
    const uint32_t k0 = kt * KT + kq;
    const uint32_t pb = k0 < P.npix ? ps_pixel(P, k0) : kOob;
#pragma unroll
    for (int i = 0; i < Q; ++i) r[i] = b.ld4(pb != kOob && toff[i] != kOob ? pb + toff[i] : kOob);
  }
};

// dW operand (ROWK, direct to LDS): rows = output channels, k = padded
// pixels of the masked gradient G_pad[b][oc][oh][OWp] (k_mask_pad).  OHWp is
// a multiple of 4, so a pixel quad is 16-byte aligned and inside one image.
struct GPadParams {
  const float* g;
  uint32_t OC, OHWp, npix, n;
  FastDiv dOHWp;
};
template <int R, int KT>
struct LdGPadRK : LoaderBase<Stage<R, KT, false>> {
  using St = Stage<R, KT, false>;
  static constexpr bool KROW = false;
  using LoaderBase<St>::Q;
  using Params = GPadParams;
  BRes b;
  GPadParams P;
  uint32_t kq;
  uint32_t ocoff[Q];
  __device__ __forceinline__ void init(const Params& p, uint32_t row0, int tid) {
    this->base_init(tid);
    P = p;
    b.init(p.g, p.n);
    kq = St::qk(tid, 0);
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t oc = row0 + St::qrow(tid, i);
      ocoff[i] = (this->act && oc < p.OC) ? oc * p.OHWp : kOob;
    }
  }
  __device__ __forceinline__ void offsets(uint32_t kt, uint32_t (&o)[Q]) const {
    const uint32_t k0 = kt * KT + kq;
    const uint32_t bb = fdiv(k0, P.dOHWp);
    const uint32_t base = k0 < P.npix ? bb * P.OC * P.OHWp + (k0 - bb * P.OHWp) : kOob;
#pragma unroll
    for (int i = 0; i < Q; ++i) o[i] = base != kOob && ocoff[i] != kOob ? base + ocoff[i] : kOob;
  }
  __device__ __forceinline__ void load(uint32_t kt, f4 (&r)[Q]) const {
    uint32_t o[Q];
    offsets(kt, o);
#pragma unroll
    for (int i = 0; i < Q; ++i) r[i] = b.ld4(o[i]);
  }
  static constexpr bool LDSD = true;
  __device__ __forceinline__ void issue_lds(uint32_t kt, float* S) const {
    if (St::PART && !this->act) return;  // whole waves (NQ is a multiple of 64)
    uint32_t o[Q];
    offsets(kt, o);
#pragma unroll
    for (int i = 0; i < Q; ++i) b.ld4_lds(o[i], S + this->wbase + i * St::DLDS);
  }
};

// ---------------------------------------------------------------------------
// Epilogues.  The accumulator layout depends on the MFMA operand order, a
// per-kernel choice (TACC, a trait of the B loader: whichever measured faster
// for that kernel's instruction schedule).  Lane l of wave (wm, wn) holds,
// for block (i, j) and register v, with r = l % 16, g = l / 16:
//   TACC false:  C[m0 + wm*16FM + 16i + 4g + v][n0 + wn*16FN + 16j + r]
//                (four consecutive rows of one column: four scalar stores);
//   TACC true:   C[m0 + wm*16FM + 16i + r][n0 + wn*16FN + 16j + 4g + v]
//                (B fragment first: four consecutive columns of one row,
//                 16 contiguous bytes of a row-major C: one quad store).
// With row-interleaved fragments (RA for the A operand, RB for B; see
// Stage::frags_rif) the wave-local row 16i + rho of fragment i becomes
// F*rho + i (frow).  RB is only used without TACC: lane (r, g) then holds FN
// consecutive columns FN*r .. FN*r + FN - 1 of each of its rows (j = 0 ..
// FN - 1), which EpiRowMajor stores as one FN-float vector.
// ---------------------------------------------------------------------------
template <bool RIF, int F>
__device__ __forceinline__ uint32_t frow(int i, int rho) {
  return RIF ? uint32_t(F * rho + i) : uint32_t(16 * i + rho);
}
__device__ __forceinline__ float epi_act(float z, uint32_t act) {
  if (act == 1) return fmaxf(z, 0.f);
  if (act == 2) return tanhf(z);
  return z;
}

struct EpiRowMajor {
  struct Params {
    float* c;
    uint32_t M, N, ldc, splitStride;
  };
  template <int MT, int NT, int FM, int FN, bool TACC, bool RA, bool RB>
  __device__ static __forceinline__ void store(const Params& p, const f4 (&acc)[FM][FN],
                                               uint32_t m0, uint32_t n0, uint32_t z, int wm,
                                               int wn, int lane) {
    float* c = p.c + size_t(z) * p.splitStride;
    const int r = lane & 15, g = lane >> 4;
    if constexpr (!TACC && RB) {
      // FN consecutive columns per row: one FN-float store (rows aligned to
      // FN floats, uniform over the launch).
      const bool vec = ((p.ldc | p.splitStride) & (FN - 1)) == 0 &&
                       (reinterpret_cast<uintptr_t>(p.c) & (4 * FN - 1)) == 0;
      const uint32_t n = n0 + wn * (FN * 16) + FN * r;
      if (n >= p.N) return;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const uint32_t m = m0 + wm * (FM * 16) + frow<RA, FM>(i, 4 * g + v);
          if (m >= p.M) continue;
          float* dst = c + size_t(m) * p.ldc + n;
          if (vec && n + FN - 1 < p.N) {
            if constexpr (FN == 4)
              *reinterpret_cast<f4*>(dst) = f4{acc[i][0][v], acc[i][1][v], acc[i][2][v], acc[i][3][v]};
            else
              *reinterpret_cast<f2*>(dst) = f2{acc[i][0][v], acc[i][1][v]};
          } else {
#pragma unroll
            for (int j = 0; j < FN; ++j)
              if (n + j < p.N) dst[j] = acc[i][j][v];
          }
        }
      }
      return;
    }
    if constexpr (!TACC) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const uint32_t n = n0 + wn * (FN * 16) + j * 16 + r;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const uint32_t m = m0 + wm * (FM * 16) + frow<RA, FM>(i, 4 * g + v);
            if (m < p.M && n < p.N) c[m * p.ldc + n] = acc[i][j][v];
          }
        }
      }
      return;
    }
    // Quad stores need 16-byte aligned rows (uniform over the launch).
    const bool vec =
        ((p.ldc | p.splitStride) & 3) == 0 && (reinterpret_cast<uintptr_t>(p.c) & 15) == 0;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const uint32_t m = m0 + wm * (FM * 16) + frow<RA, FM>(i, r);
      if (m >= p.M) continue;
      float* row = c + size_t(m) * p.ldc;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const uint32_t n = n0 + wn * (FN * 16) + j * 16 + 4 * g;
        if (vec && n + 3 < p.N) {
          *reinterpret_cast<f4*>(row + n) = acc[i][j];
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v)
            if (n + v < p.N) row[n + v] = acc[i][j][v];
        }
      }
    }
  }
};

// NCHW output: out[b][m][pix] for n = b*HW + pix; optional bias + activation
// (0 identity, 1 ReLU, 2 tanh), as nn_conv_reshape.hlsl:23-26.  With TACC a
// lane's four columns are four consecutive pixels of one plane unless they
// cross an image boundary; the quad is stored at 4-byte alignment (planes of
// odd size; unaligned access is on).
struct EpiNCHW {
  struct Params {
    float* out;
    const float* bias;
    uint32_t M, HW, N, act;
    FastDiv dHW;
  };
  template <int MT, int NT, int FM, int FN, bool TACC, bool RA, bool RB>
  __device__ static __forceinline__ void store(const Params& p, const f4 (&acc)[FM][FN],
                                               uint32_t m0, uint32_t n0, uint32_t, int wm,
                                               int wn, int lane) {
    const int r = lane & 15, g = lane >> 4;
    if constexpr (!TACC) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const uint32_t n = n0 + wn * (FN * 16) + frow<RB, FN>(j, r);
        const uint32_t b = fdiv(n, p.dHW);
        const uint32_t base = b * p.M * p.HW + (n - b * p.HW);
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const uint32_t m = m0 + wm * (FM * 16) + frow<RA, FM>(i, 4 * g + v);
            if (m < p.M && n < p.N)
              p.out[base + m * p.HW] = epi_act(acc[i][j][v] + (p.bias ? p.bias[m] : 0.f), p.act);
          }
        }
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const uint32_t n = n0 + wn * (FN * 16) + j * 16 + 4 * g;
      if (n >= p.N) continue;
      const uint32_t b = fdiv(n, p.dHW);
      const uint32_t pix = n - b * p.HW;
      const bool quad = pix + 3 < p.HW && n + 3 < p.N;
      const size_t base = size_t(b) * p.M * p.HW + pix;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const uint32_t m = m0 + wm * (FM * 16) + frow<RA, FM>(i, r);
        if (m >= p.M) continue;
        const float bias = p.bias ? p.bias[m] : 0.f;
        f4 z;
#pragma unroll
        for (int v = 0; v < 4; ++v) z[v] = epi_act(acc[i][j][v] + bias, p.act);
        if (quad) {
          stu(p.out + base + size_t(m) * p.HW, z);
        } else {
          uint32_t bb = b, pp = pix;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            if (n + v < p.N) p.out[(size_t(bb) * p.M + m) * p.HW + pp] = z[v];
            if (++pp == p.HW) {
              pp = 0;
              ++bb;
            }
          }
        }
      }
    }
  }
};

// NCHW output over a padded pixel grid (n = b*OHWp + oh*OWp + ow, ow < OWp,
// OWp % 4 == 0, so a TACC lane's four columns share one padded row): columns
// with ow >= OW are dropped; otherwise as EpiNCHW.
struct EpiNCHWPad {
  struct Params {
    float* out;
    const float* bias;
    uint32_t M, OHW, OW, OWp, OHWp, N, act;
    FastDiv dOHWp, dOWp;
  };
  template <int MT, int NT, int FM, int FN, bool TACC, bool RA, bool RB>
  __device__ static __forceinline__ void store(const Params& p, const f4 (&acc)[FM][FN],
                                               uint32_t m0, uint32_t n0, uint32_t, int wm,
                                               int wn, int lane) {
    static_assert(!(TACC && RB), "row-interleaved B fragments are not used with TACC");
    const int r = lane & 15, g = lane >> 4;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const uint32_t n = n0 + wn * (FN * 16) + (TACC ? j * 16 + 4 * g : frow<RB, FN>(j, r));
      const uint32_t b = fdiv(n, p.dOHWp), rem = n - b * p.OHWp;
      const uint32_t oh = fdiv(rem, p.dOWp), ow = rem - oh * p.OWp;
      if (n >= p.N || ow >= p.OW) continue;
      const size_t base = size_t(b) * p.M * p.OHW + oh * p.OW + ow;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        if constexpr (!TACC) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const uint32_t m = m0 + wm * (FM * 16) + frow<RA, FM>(i, 4 * g + v);
            if (m < p.M)
              p.out[base + size_t(m) * p.OHW] =
                  epi_act(acc[i][j][v] + (p.bias ? p.bias[m] : 0.f), p.act);
          }
        } else {
          const uint32_t m = m0 + wm * (FM * 16) + frow<RA, FM>(i, r);
          if (m >= p.M) continue;
          const float bias = p.bias ? p.bias[m] : 0.f;
          f4 z;
#pragma unroll
          for (int v = 0; v < 4; ++v) z[v] = epi_act(acc[i][j][v] + bias, p.act);
          float* dst = p.out + base + size_t(m) * p.OHW;
          if (ow + 3 < p.OW) {
            stu(dst, z);
          } else {
#pragma unroll
            for (int v = 0; v < 4; ++v)
              if (ow + v < p.OW) dst[v] = z[v];
          }
        }
      }
    }
  }
};

// One sub-pixel phase of a strided dX: columns n = b*GHW + a*GW + c of the
// phase's pixel grid go to out[b][m][ph + s*a][pw + s*c] (NCHW, H x W
// planes).  Consecutive columns land s floats apart, so every value is its
// own store.
struct EpiNCHWPhase {
  struct Params {
    float* out;
    uint32_t M, H, W, GW, GHW, N, s, ph, pw;
    FastDiv dGHW, dGW;
  };
  __device__ static __forceinline__ size_t at(const Params& p, uint32_t n, uint32_t m) {
    const uint32_t b = fdiv(n, p.dGHW), rem = n - b * p.GHW;
    const uint32_t a = fdiv(rem, p.dGW), c = rem - a * p.GW;
    return (size_t(b) * p.M + m) * p.H * p.W + size_t(p.ph + p.s * a) * p.W + p.pw + p.s * c;
  }
  template <int MT, int NT, int FM, int FN, bool TACC, bool RA, bool RB>
  __device__ static __forceinline__ void store(const Params& p, const f4 (&acc)[FM][FN],
                                               uint32_t m0, uint32_t n0, uint32_t, int wm,
                                               int wn, int lane) {
    static_assert(!(TACC && RB), "row-interleaved B fragments are not used with TACC");
    const int r = lane & 15, g = lane >> 4;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          // TACC: row 16i + r, column 16j + 4g + v; else row 16i + 4g + v, column 16j + r
          const uint32_t m = m0 + wm * (FM * 16) + (TACC ? frow<RA, FM>(i, r) : frow<RA, FM>(i, 4 * g + v));
          const uint32_t n = n0 + wn * (FN * 16) + (TACC ? j * 16 + 4 * g + v : frow<RB, FN>(j, r));
          if (m < p.M && n < p.N) p.out[at(p, n, m)] = acc[i][j][v];
        }
  }
};

// EpiNCHW that also leaves the batch-norm statistics of the values it stores:
// for each output row m (a channel) the sums of z and z*z over the tile's
// columns below N, as doubles at stats[(m * pieces + nt) * 2 + {0, 1}] with
// nt the tile's column index: one piece per column tile, the layout of the
// BN statistics' partial sums.  The transposed-accumulation form only (the
// pixel and pointwise GEMMs): a lane's row is fixed per fragment, so it
// stores each quad as EpiNCHW does and adds its (at most 16) values of the
// row in float; the lanes' float pairs go to LDS (the A stages, free after
// the main loop's last barrier) and after one barrier a thread per row adds
// them in double in a fixed order (the same bits on every run).  The row's
// bias is loaded once for both uses.
struct EpiNCHWStats {
  static constexpr bool kStats = true;
  struct Params {
    EpiNCHW::Params o;
    double* stats;
    uint32_t pieces;
  };
  // All WGN waves of the workgroup call this.  lds: WGN * 4 * MT float2.
  template <int MT, int NT, int FM, int FN, bool TACC, bool RA, bool RB, int WGN>
  __device__ static __forceinline__ void store_stats(const Params& p, const f4 (&acc)[FM][FN],
                                                     uint32_t m0, uint32_t n0, int wm, int wn,
                                                     int lane, float* lds) {
    static_assert(TACC && WGN > 1, "pixel-column GEMMs with several waves per row block");
    const EpiNCHW::Params& o = p.o;
    const int r = lane & 15, g = lane >> 4;
    float2* red = reinterpret_cast<float2*>(lds);
    uint32_t m[FM];
    float bv[FM], f0[FM], f1[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      m[i] = m0 + wm * (FM * 16) + frow<RA, FM>(i, r);
      bv[i] = o.bias && m[i] < o.M ? o.bias[m[i]] : 0.f;
      f0[i] = f1[i] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const uint32_t n = n0 + wn * (FN * 16) + j * 16 + 4 * g;
      const uint32_t b = fdiv(n, o.dHW);
      const uint32_t pix = n - b * o.HW;
      const bool quad = pix + 3 < o.HW && n + 3 < o.N;
      const size_t base = size_t(b) * o.M * o.HW + pix;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        f4 z;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          z[v] = epi_act(acc[i][j][v] + bv[i], o.act);
          const float zz = m[i] < o.M && n + v < o.N ? z[v] : 0.f;
          f0[i] += zz;
          f1[i] = fmaf(zz, zz, f1[i]);
        }
        if (m[i] >= o.M || n >= o.N) continue;
        if (quad) {
          stu(o.out + base + size_t(m[i]) * o.HW, z);
        } else {
          uint32_t bb = b, pp = pix;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            if (n + v < o.N) o.out[(size_t(bb) * o.M + m[i]) * o.HW + pp] = z[v];
            if (++pp == o.HW) {
              pp = 0;
              ++bb;
            }
          }
        }
      }
    }
    // Lane (r, g) of wave (wm, wn) holds row wm*WM + frow(i, r): slot
    // (wn * 4 + g) of that row.
#pragma unroll
    for (int i = 0; i < FM; ++i)
      red[(wn * 4 + g) * MT + wm * (FM * 16) + frow<RA, FM>(i, r)] = float2{f0[i], f1[i]};
    __syncthreads();
    const int t = threadIdx.x;
    if (t < MT && m0 + t < o.M) {
      double s0 = 0, s1 = 0;
#pragma unroll
      for (int w = 0; w < WGN * 4; ++w) {
        const float2 e = red[w * MT + t];
        s0 += double(e.x);
        s1 += double(e.y);
      }
      double* d = p.stats + (size_t(m0 + t) * p.pieces + n0 / NT) * 2;
      d[0] = s0;
      d[1] = s1;
    }
  }
};
template <class E, class = void>
struct EpiStats : std::false_type {};
template <class E>
struct EpiStats<E, std::void_t<decltype(E::kStats)>> : std::true_type {};

// ---------------------------------------------------------------------------
// The kernel.
// ---------------------------------------------------------------------------
// Tile order.  The dispatcher hands consecutive workgroup ids to the eight
// XCDs in turn, and each XCD has its own L2.  With `xcd` set, the ids are
// renumbered so that each XCD receives a contiguous run of logical tiles; the
// logical order is m-tile fastest, then n-tile, then split, so the tiles that
// read the same operand rows (the same n-tile, or the same split's K range)
// run on one XCD at about the same time.
struct TileGrid {
  uint32_t gm, gn, xcd;
};
__device__ __forceinline__ void tile_coords(const TileGrid& tg, uint32_t& mt, uint32_t& nt,
                                            uint32_t& z) {
  const uint32_t id = tg.xcd ? xcd_block_id() : blockIdx.x;
  mt = id % tg.gm;
  const uint32_t t = id / tg.gm;
  nt = t % tg.gn;
  z = t / tg.gn;
}

// Occupancy floor: the 128 x 128 tile holds 64 accumulator registers per
// lane, and four workgroups per CU (the LDS limit) need the rest of the
// register file to fit in 64 more.
template <int MT, int NT>
constexpr int igemm_min_waves() {
  return MT * NT == 128 * 128 ? 4 : (MT * NT == 256 * 128 ? 2 : 1);
}

template <int MT, int NT, int KT, class LA, class LB, class EPI>
__global__ void __launch_bounds__(kThreads)
    __attribute__((amdgpu_waves_per_eu(igemm_min_waves<MT, NT>())))
    k_igemm(const typename LA::Params pa, const typename LB::Params pb,
            const typename EPI::Params pe, TileGrid tg, uint32_t ktiles, uint32_t splits) {
  using SA = typename LA::St;
  using SB = typename LB::St;
  // WKS (narrow tiles, MT <= 32 with KT = 64): the four waves split every K
  // tile, each computing the whole MT x NT tile over its own 16-k slice, and
  // the four partial tiles are added in wave order at the end.  A barrier
  // then covers four times the MFMA work of the 1 x 4 wave grid at KT = 16.
  constexpr bool WKS = MT <= 32 && KT == 64;
  constexpr int WGM = WKS ? 1 : (MT >= 64 ? 2 : 1), WGN = WKS ? 1 : 4 / WGM;  // wave grid
  constexpr int WM = MT / WGM, WN = NT / WGN, FM = WM / 16, FN = WN / 16;
  static_assert(FM >= 1 && FN >= 1 && WM % 16 == 0 && WN % 16 == 0, "tile too small");
  __shared__ __attribute__((aligned(16))) float As[2 * SA::SIZE];
  __shared__ __attribute__((aligned(16))) float Bs[2 * SB::SIZE];
  static_assert(!WKS || 3 * FM * FN * 256 <= 2 * SB::SIZE, "wave partials fit the B stages");

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = WKS ? 0 : wave / WGN, wn = WKS ? 0 : wave % WGN;  // WKS: every wave the whole tile
  uint32_t mt, nt, z;
  tile_coords(tg, mt, nt, z);
  const uint32_t m0 = mt * MT, n0 = nt * NT;
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

  constexpr bool DA = LA::LDSD, DB = LB::LDSD;
  constexpr bool TACC = LB::kTransAcc;
  // Row-interleaved fragments for [k][row] operands read 2 or 4 fragments at
  // a time (B only without TACC, whose quad stores need 16-row fragments).
  constexpr bool RA = SA::kRow && (FM == 2 || FM == 4);
  constexpr bool RB = SB::kRow && !TACC && (FN == 2 || FN == 4);
  const int r = lane & 15, g = lane >> 4;
  // Fragments of one 16-deep k slice of LDS stage `cur`, and its MFMAs.
  struct Frags {
    f4 a[FM], b[FN];
  };
  auto read_slice = [&](int cur, int ks, Frags& f) {
    const float* Ac = As + cur * SA::SIZE;
    const float* Bc = Bs + cur * SB::SIZE;
    if constexpr (RA) {
      SA::template frags_rif<FM>(Ac, wm * WM, r, g, ks, f.a);
    } else {
#pragma unroll
      for (int i = 0; i < FM; ++i) f.a[i] = SA::frag(Ac, wm * WM + i * 16, r, g, ks);
    }
    if constexpr (RB) {
      SB::template frags_rif<FN>(Bc, wn * WN, r, g, ks, f.b);
    } else {
#pragma unroll
      for (int j = 0; j < FN; ++j) f.b[j] = SB::frag(Bc, wn * WN + j * 16, r, g, ks);
    }
  };
  auto mfma_slice = [&](const Frags& f) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          // TACC: B first, the block accumulates C transposed (see the epilogues).
          acc[i][j] = TACC ? __builtin_amdgcn_mfma_f32_16x16x4f32(f.b[j][s], f.a[i][s], acc[i][j], 0, 0, 0)
                           : __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[i][s], f.b[j][s], acc[i][j], 0, 0, 0);
  };
  if (kb < ke) {
    if constexpr (DA) la.issue_lds(kb, As); else la.load(kb, ra);
    if constexpr (DB) lb.issue_lds(kb, Bs); else lb.load(kb, rb);
    if constexpr (!DA) la.store(As, ra);
    if constexpr (!DB) lb.store(Bs, rb);
  }
  if constexpr (DA || DB) __builtin_amdgcn_s_waitcnt(0);  // the direct loads have landed
  __syncthreads();

  for (uint32_t kt = kb; kt < ke; ++kt) {
    const int cur = int(kt - kb) & 1;
    const bool more = kt + 1 < ke;
    // The first slice's fragments are read before the next tile's loads are
    // issued: a direct load into LDS that is still in flight would otherwise
    // make the compiler wait for it before any LDS read.
    Frags f0;
    read_slice(cur, WKS ? 16 * wave : 0, f0);
    // Next tile: register staging, or straight into the other LDS stage (its
    // readers finished before the previous barrier).
    if (more) {
      if constexpr (DA) la.issue_lds(kt + 1, As + (cur ^ 1) * SA::SIZE); else la.load(kt + 1, ra);
      if constexpr (DB) lb.issue_lds(kt + 1, Bs + (cur ^ 1) * SB::SIZE); else lb.load(kt + 1, rb);
    }
    mfma_slice(f0);
    if constexpr (!WKS) {
#pragma unroll
      for (int ks = 16; ks < KT; ks += 16) {
        Frags f;
        read_slice(cur, ks, f);
        mfma_slice(f);
      }
    }
    // Every MFMA of the tile is issued before the wait for the next tile's
    // loads and the barrier (the scheduler would otherwise hoist them above
    // part of the MFMAs, and a wave would stall on the loads with MFMA work
    // still unissued).
    __builtin_amdgcn_sched_barrier(0);
    if (more) {
      if constexpr (!DA) la.store(As + (cur ^ 1) * SA::SIZE, ra);
      if constexpr (!DB) lb.store(Bs + (cur ^ 1) * SB::SIZE, rb);
    }
    if constexpr (DA || DB) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  if constexpr (WKS) {
    // Waves 1-3 park their partial tiles in the (now idle) B stages; wave 0
    // adds them in wave order and stores the tile.
    f4* red = reinterpret_cast<f4*>(Bs);
    if (wave != 0) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) red[((wave - 1) * FM * FN + i * FN + j) * 64 + lane] = acc[i][j];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < 3; ++w)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] += red[(w * FM * FN + i * FN + j) * 64 + lane];
  }
  if constexpr (EpiStats<EPI>::value) {
    static_assert(WGN * 4 * MT * 8 <= int(sizeof(As)), "the statistics' lane sums fit the A stages");
    EPI::template store_stats<MT, NT, FM, FN, TACC, RA, RB, WGN>(pe, acc, m0, n0, wm, wn, lane, As);
  } else {
    EPI::template store<MT, NT, FM, FN, TACC, RA, RB>(pe, acc, m0, n0, z, wm, wn, lane);
  }
}

// ---------------------------------------------------------------------------
// Side kernels: NHWC transpose (+ ReLU mask + bias-gradient partials),
// filter re-layouts, split-K sums.
// ---------------------------------------------------------------------------
// Filters in the K order of the pixel loaders (flat or blocked), zero for
// padding channels; `inner` is the padded channel count the K axis runs over
// (Cp for the forward, OCp for dX):
// mode 0 (forward A): out[oc][kk] = w[oc][c][khw]   with c  = channel of kk
// mode 1 (dX A):      out[c][kk]  = w[oc][c][khw]   with oc = channel of kk
// where kk = khw*inner + ch (flat) or (cb*KK + khw)*kCB + ci, ch = cb*kCB + ci
// (blocked).  Rows are ld >= KK*inner floats apart, zero past KK*inner; size
// rows * ld, rows = OC (mode 0) or C (mode 1).  The packed forward (C < 4
// channels) uses the flat order with inner = C and ld = pad4(KK*C).
// With vw != 0 the K order runs over the taps of one sub-pixel phase of a
// strided dX: virtual tap v = jh * vw + jw is the filter tap (rh + s*jh,
// rw + s*jw) of a kk x kk filter, and KK counts the phase's taps.
struct WPerm {
  const float* w;  // null: nothing to re-lay
  float* out;
  uint32_t OC, C, KK, inner, ld;
  int mode, blocked;
  uint32_t vw, kk, s, rh, rw;
  uint32_t blocks() const { return w ? cdiv(size_t(mode == 0 ? OC : C) * ld, 256) : 0; }
};

__device__ __forceinline__ void permute_w_elem(const WPerm& pw, uint32_t i) {
  const float* __restrict__ w = pw.w;
  float* __restrict__ out = pw.out;
  const uint32_t OC = pw.OC, C = pw.C, KK = pw.KK, inner = pw.inner, ld = pw.ld;
  const int mode = pw.mode, blocked = pw.blocked;
  const uint32_t kdim = KK * inner;
  const uint32_t rows = mode == 0 ? OC : C;
  if (i >= rows * ld) return;
  const uint32_t r = i / ld, kk = i - r * ld;
  if (kk >= kdim) {  // row pitch padding
    out[i] = 0.f;
    return;
  }
  uint32_t khw, ch;
  if (blocked) {
    const uint32_t blk = kk / kCB, ci = kk - blk * kCB;
    const uint32_t cb = blk / KK;
    khw = blk - cb * KK;
    ch = cb * kCB + ci;
  } else {
    khw = kk / inner;
    ch = kk - khw * inner;
  }
  uint32_t wk = khw, wKK = KK;
  if (pw.vw) {
    const uint32_t jh = khw / pw.vw, jw = khw - jh * pw.vw;
    wk = (pw.rh + pw.s * jh) * pw.kk + pw.rw + pw.s * jw;
    wKK = pw.kk * pw.kk;
  }
  if (mode == 0)
    out[i] = ch < C ? w[(r * C + ch) * wKK + wk] : 0.f;
  else
    out[i] = ch < OC ? w[(ch * C + r) * wKK + wk] : 0.f;
}

__global__ void k_permute_w(WPerm pw) { permute_w_elem(pw, blockIdx.x * blockDim.x + threadIdx.x); }

static bool permute_w(const WPerm& pw) {
  hipLaunchKernelGGL(k_permute_w, dim3(pw.blocks()), dim3(256), 0, stream(), pw);
  return check_launch("permute_w");
}

// out[((b*HW) + p)*Cp + c] = (c < C) ? in[(b*C + c)*HW + p] masked : 0.
// Block: CB channels x PB = 2048 / CB pixels through LDS (CB = 16 for tensors
// of at most 16 channels, 32 otherwise, so few-channel tensors do not leave
// half the block idle).  dbPart[c][b*npb + block]: the masked values of
// channel c summed over the block's pixels.
// Loads are 16-byte quads of 4 pixels of one channel row and stores 16-byte
// quads of 4 channels of one pixel (Cp % 4 == 0 keeps those aligned).  Plane
// rows of odd length leave the load quads only 4-byte aligned; the GPU runs
// with unaligned access enabled.  A quad that would cross the end of its row
// is read dword by dword.
// Workgroups past the first nMain re-lay filters instead (pw: the forward's
// filter permutation, which then costs no launch of its own).
// BNDX: `in` is the dy of a batch norm and `y` its input x; the values
// transposed are that batch norm's dx (bn_dx_elem), which the kernel also
// stores in NCHW to bn.dx: batchnorm_backward_dx and the transpose pass of
// the conv below it in one pass.
struct BnDxArgs {
  const float* mean;
  const float* var;
  const float* gamma;
  const float* dg;
  const float* db;
  float* dx;
  float eps, m;
};
template <int CB, bool BNDX = false>
__global__ void __launch_bounds__(256)
    k_to_nhwc(const float* __restrict__ in, const float* __restrict__ y, float* __restrict__ out,
              float* __restrict__ dbPart, uint32_t C, uint32_t HW, uint32_t Cp, uint32_t npb,
              uint32_t ncb, uint32_t nB, uint32_t nMain, WPerm pw, BnDxArgs bn = BnDxArgs{}) {
  if (blockIdx.x >= nMain) {
    permute_w_elem(pw, (blockIdx.x - nMain) * 256 + threadIdx.x);
    return;
  }
  constexpr int PB = 2048 / CB, PQ = PB / 4;  // pixels per block, pixel quads per row
  constexpr int CR = 256 / PQ;                // channel rows per load pass
  constexpr int PR = 256 / (CB / 4);          // pixels per store pass
  static_assert(CR * 2 == CB && PR * 2 == PB, "two load and two store passes");
  __shared__ float t[CB][PB + 1];
  // 1-D grid over (pixel block, channel block, image), pixel block fastest,
  // in XCD-contiguous order: a plane row's neighbouring blocks share its
  // partial cache lines.
  const uint32_t id = xcd_block_id(nMain);
  const uint32_t pb = id % npb, rest = id / npb;
  const uint32_t c0 = (rest % ncb) * CB, p0 = pb * PB, b = rest / ncb;
  const int tid = threadIdx.x;
  // Branch-free loads through buffer resources (elements outside the tile's
  // channels / pixels read at kOob, i.e. zero): all of a thread's loads are
  // in flight together.  Callers admit tensors below kOob floats.
  BRes bi, by;
  const uint32_t n = nB * C * HW;
  bi.init(in, n);
  by.init(y ? y : in, n);
  const int pq = tid % PQ;  // pixel quad of the load phase
  f4 v[2], m[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t c = c0 + tid / PQ + CR * j, p = p0 + 4 * pq;
    const uint32_t row = (b * C + c) * HW;
    if (c < C && p + 3 < HW) {
      v[j] = bi.ld4(row + p);
      m[j] = y ? by.ld4(row + p) : f4{1.f, 1.f, 1.f, 1.f};
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t off = (c < C && p + e < HW) ? row + p + e : kOob;
        v[j][e] = bi.ld1(off);
        m[j][e] = y ? by.ld1(off) : 1.f;
      }
    }
  }
  if constexpr (BNDX) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t c = c0 + tid / PQ + CR * j, p = p0 + 4 * pq;
      if (c >= C) {
        v[j] = zero4();
        continue;
      }
      const float mu = bn.mean[c], rstd = 1.0f / sqrtf(bn.var[c] + bn.eps);
      const float g = bn.gamma[c], dg = bn.dg[c], db = bn.db[c];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[j][e] = p + e < HW ? bn_dx_elem(m[j][e], v[j][e], mu, rstd, g, dg, db, bn.m) : 0.f;
      float* dst = bn.dx + (size_t(b) * C + c) * HW + p;
      if (p + 3 < HW) {
        stu(dst, v[j]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (p + e < HW) dst[e] = v[j][e];
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) t[tid / PQ + CR * j][4 * pq + e] = v[j][e];
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        // ReLU mask: y <= 0 zeroes the gradient (a NaN y keeps it).
        t[tid / PQ + CR * j][4 * pq + e] = m[j][e] <= 0.f ? 0.f : v[j][e];
  }
  __syncthreads();
  if (dbPart != nullptr && tid < 8 * CB) {
    // 8 lanes per channel, PB / 8 pixels each, then a fixed butterfly.
    const int cl = tid >> 3, part = tid & 7;
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < PB / 8; ++q) s += t[cl][part * (PB / 8) + q];
    s = group8_reduce(s);
    if (part == 0 && c0 + cl < C)
      dbPart[size_t(c0 + cl) * nB * npb + size_t(b) * npb + pb] = s;
  }
  const int cq = tid % (CB / 4);  // channel quad of the store phase
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int pl = tid / (CB / 4) + PR * j;
    const uint32_t c = c0 + 4 * cq, p = p0 + pl;
    const f4 q = {t[4 * cq][pl], t[4 * cq + 1][pl], t[4 * cq + 2][pl], t[4 * cq + 3][pl]};
    if (p < HW && c < Cp) *reinterpret_cast<f4*>(out + (size_t(b) * HW + p) * Cp + c) = q;
  }
}

// Few channels (Cp <= 8): one thread per pixel reads its C channel values
// (coalesced across threads per channel) and stores Cp/4 quads.
__global__ void k_to_nhwc_small(const float* __restrict__ in, float* __restrict__ out, uint32_t C,
                                uint32_t HW, uint32_t Cp, uint32_t npix, FastDiv dHW) {
  const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= npix) return;
  const uint32_t b = fdiv(n, dHW), p = n - b * HW;
  const float* src = in + size_t(b) * C * HW + p;
  f4* dst = reinterpret_cast<f4*>(out + size_t(n) * Cp);
  for (uint32_t q = 0; q < Cp / 4; ++q) {
    f4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = (4 * q + e < C) ? src[size_t(4 * q + e) * HW] : 0.f;
    dst[q] = v;
  }
}

// out[c] = sum of the `rows` partials of channel c (stored contiguously,
// part[c*rows + r]): 256 strided per-thread sums, then a fixed tree.  One
// 256-thread block per channel.
__device__ __forceinline__ void rowsum_block(const float* __restrict__ part,
                                             float* __restrict__ out, uint32_t rows,
                                             uint32_t c) {
  __shared__ float sh[4];
  const float* p = part + size_t(c) * rows;
  float s = 0.f;
#pragma unroll 8
  for (uint32_t r = threadIdx.x; r < rows; r += 256) s += p[r];
  s = wave_reduce(s);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) out[c] = (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

__global__ void __launch_bounds__(256)
    k_rowsum(const float* __restrict__ part, float* __restrict__ out, uint32_t rows) {
  rowsum_block(part, out, rows, blockIdx.x);
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

// Quad form of k_splitk_sum for n % 4 == 0 (same summation order).
// Sum of the split partials p[0], p[zs], p[2 zs], ... in split order; the
// loads of each group of up to four are issued before its adds (the finishes
// run at 2 - 3 splits, which a one-at-a-time loop would serialise).
__device__ __forceinline__ f4 sum_splits4(const f4* __restrict__ p, size_t zs, uint32_t splits) {
  f4 s = {0.f, 0.f, 0.f, 0.f};
  uint32_t z = 0;
  for (; z + 3 < splits; z += 4) {
    const f4 a = p[z * zs], b = p[(z + 1) * zs], c = p[(z + 2) * zs], d = p[(z + 3) * zs];
    s += a;
    s += b;
    s += c;
    s += d;
  }
  const uint32_t rem = splits - z;  // uniform across the grid
  if (rem == 3) {
    const f4 a = p[z * zs], b = p[(z + 1) * zs], c = p[(z + 2) * zs];
    s += a;
    s += b;
    s += c;
  } else if (rem == 2) {
    const f4 a = p[z * zs], b = p[(z + 1) * zs];
    s += a;
    s += b;
  } else if (rem == 1) {
    s += p[z * zs];
  }
  return s;
}
__global__ void __launch_bounds__(256)
    k_splitk_sum4(const f4* __restrict__ part, f4* __restrict__ out, uint32_t nq,
                  uint32_t splits) {
  const uint32_t q = blockIdx.x * 256 + threadIdx.x;
  if (q >= nq) return;
  out[q] = sum_splits4(part + q, nq, splits);
}

// dW finalize: dw[oc][c][khw] = sum_z part[z][oc][khw*Cp + c], or with
// `trans` (the GEMM ran with taps as rows) sum_z part[z][khw*Cp + c][oc].
// Quad form: thread (quad q, slice w) sums the 16-byte quads part[z][4q..]
// over z = w, w + SL, w + 2 SL, ... (four loads in flight); with SL > 1 the
// SL slice sums are then added in slice order through LDS, so the result is
// deterministic.  SL (1, 4 or 16) is chosen from the quad count alone, which
// keeps enough loads in flight when few quads take many splits.  Elements
// i = 4q + j are stored in storage order of the partials; Cp is the channel
// stride of the tap axis (pad4(C), or C for the packed layout), and each
// split's partials start 4 * ceil(OC*KK*Cp / 4) floats apart.  Padding
// channels (c >= C) and the tail past OC*KK*Cp are dropped.
//
// The same launch carries the conv backward's bias-gradient sum as side.nRow
// extra blocks after the nMain finishing blocks (rowsum_block), so that it
// costs no launch of its own; the two jobs touch disjoint buffers.
struct BwdSide {
  const float* dbPart;  // bias-gradient partials [OC][dbRows]
  float* db;
  uint32_t dbRows, nRow;  // nRow = OC, or 0 for no bias gradient
};

// dbCol (not null, KK == 1, !trans): the tap axis' column C holds the bias
// gradient (a GEMM operand row of ones), written to dbCol[oc].
template <int SL>
__global__ void __launch_bounds__(256)
    k_dw_final(const f4* __restrict__ part, float* __restrict__ dw, uint32_t OC, uint32_t C,
               uint32_t KK, uint32_t Cp, uint32_t splits, uint32_t trans, uint32_t nMain,
               BwdSide side, float* __restrict__ dbCol, WPerm pw) {
  if (blockIdx.x >= nMain) {
    // Extra blocks: the bias-gradient sum (one per channel), then a filter
    // re-layout riding in this launch.
    const uint32_t e = blockIdx.x - nMain;
    if (e < side.nRow)
      rowsum_block(side.dbPart, side.db, side.dbRows, e);
    else
      permute_w_elem(pw, (e - side.nRow) * 256 + threadIdx.x);
    return;
  }
  constexpr uint32_t QB = 256 / SL;
  __shared__ f4 sh[SL][QB];
  const uint32_t N = KK * Cp, total = OC * N, nq = (total + 3) / 4;
  const uint32_t lq = threadIdx.x % QB, w = threadIdx.x / QB;
  const uint32_t q = blockIdx.x * QB + lq;
  f4 s = {0.f, 0.f, 0.f, 0.f};
  if (q < nq) {
    const size_t zs = nq;
    uint32_t z = w;
    // Eight loads in flight, added in z order.
    for (; z + 7 * SL < splits; z += 8 * SL) {
      f4 t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = part[(z + u * SL) * zs + q];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += t[u];
    }
    for (; z + 3 * SL < splits; z += 4 * SL) {
      const f4 a = part[z * zs + q], b = part[(z + SL) * zs + q];
      const f4 c = part[(z + 2 * SL) * zs + q], d = part[(z + 3 * SL) * zs + q];
      s += a;
      s += b;
      s += c;
      s += d;
    }
    for (; z < splits; z += SL) s += part[z * zs + q];
  }
  if constexpr (SL > 1) {
    sh[w][lq] = s;
    __syncthreads();
    if (w != 0) return;
    s = sh[0][lq];
#pragma unroll
    for (int k = 1; k < SL; ++k) s += sh[k][lq];
  }
  if (q >= nq) return;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t i = 4 * q + j;
    if (i >= total) break;
    uint32_t oc, n;
    if (trans) {
      n = i / OC;
      oc = i - n * OC;
    } else {
      oc = i / N;
      n = i - oc * N;
    }
    const uint32_t khw = n / Cp, c = n - khw * Cp;
    if (c < C)
      dw[(size_t(oc) * C + c) * KK + khw] = s[j];
    else if (dbCol && c == C)
      dbCol[oc] = s[j];
  }
}

// Slices per quad for k_dw_final: the fewest (1, 4, 16) that give about
// 128 K threads, never more than the splits.
static uint32_t dw_final_slices(uint32_t nq, uint32_t splits) {
  uint32_t sl = 1;
  while (sl < 16 && size_t(nq) * sl < 131072 && sl * 4 <= splits) sl *= 4;
  return sl;
}

static bool dw_final(const float* part, float* dw, uint32_t OC, uint32_t C, uint32_t KK,
                     uint32_t Cp, uint32_t splits, bool trans, BwdSide side = BwdSide{},
                     float* dbCol = nullptr, const WPerm& pw = WPerm{}) {
  const uint32_t nq = cdiv(size_t(OC) * KK * Cp, 4), sl = dw_final_slices(nq, splits);
  const f4* p4 = reinterpret_cast<const f4*>(part);
  const uint32_t tr = trans ? 1u : 0u;
  const uint32_t nMain = cdiv(nq, 256u / sl);
  const dim3 grid(nMain + side.nRow + pw.blocks());
  if (sl == 1)
    hipLaunchKernelGGL(k_dw_final<1>, grid, dim3(256), 0, stream(), p4, dw, OC, C, KK, Cp, splits,
                       tr, nMain, side, dbCol, pw);
  else if (sl == 4)
    hipLaunchKernelGGL(k_dw_final<4>, grid, dim3(256), 0, stream(), p4, dw, OC, C, KK, Cp, splits,
                       tr, nMain, side, dbCol, pw);
  else
    hipLaunchKernelGGL(k_dw_final<16>, grid, dim3(256), 0, stream(), p4, dw, OC, C, KK, Cp,
                       splits, tr, nMain, side, dbCol, pw);
  return check_launch("dw_final");
}

// Split-K finish for an NCHW output: out[b][m][pix] = act(sum_z part[z][m][n]
// + bias[m]) for n = b*HW + pix, z summed in order (deterministic).
__global__ void k_splitk_nchw(const float* __restrict__ part, const float* __restrict__ bias,
                              float* __restrict__ out, uint32_t M, uint32_t N, uint32_t HW,
                              uint32_t splits, uint32_t act) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * N) return;
  const uint32_t m = i / N, n = i - m * N;
  float z = 0.f;
  for (uint32_t k = 0; k < splits; ++k) z += part[size_t(k) * M * N + i];
  if (bias) z += bias[m];
  if (act == 1)
    z = fmaxf(z, 0.f);
  else if (act == 2)
    z = tanhf(z);
  const uint32_t b = n / HW, pix = n - b * HW;
  out[(size_t(b) * M + m) * HW + pix] = z;
}

// Quad form of k_splitk_nchw for N % 4 == 0: 16-byte partial loads, four in
// flight, z still summed in order (same bits as the scalar form).  The four
// elements of a quad lie in one row m and may straddle an image boundary.
__global__ void __launch_bounds__(256)
    k_splitk_nchw4(const f4* __restrict__ part, const float* __restrict__ bias,
                   float* __restrict__ out, uint32_t M, uint32_t N, uint32_t HW, uint32_t splits,
                   uint32_t act) {
  const uint32_t q = blockIdx.x * 256 + threadIdx.x;
  const uint32_t nq = M * (N / 4);
  if (q >= nq) return;
  f4 s = sum_splits4(part + q, nq, splits);
  const uint32_t m = (4 * q) / N, n0 = 4 * q - m * N;
  uint32_t b = n0 / HW, pix = n0 - b * HW;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v = s[j];
    if (bias) v += bias[m];
    if (act == 1)
      v = fmaxf(v, 0.f);
    else if (act == 2)
      v = tanhf(v);
    s[j] = v;
  }
  if (pix + 3 < HW) {
    // The quad lies in one plane: one 16-byte store (4-byte aligned for planes
    // of odd size; unaligned access is on).
    stu(out + (size_t(b) * M + m) * HW + pix, s);
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    out[(size_t(b) * M + m) * HW + pix] = s[j];
    if (++pix == HW) {
      pix = 0;
      ++b;
    }
  }
}

// k_splitk_nchw that also leaves the batch-norm statistics of what it
// stores (as EpiNCHWStats): block (piece, m) finishes columns
// [piece * kStatsSpan, (piece + 1) * kStatsSpan) of row m, with the same sum
// order as k_splitk_nchw / k_splitk_nchw4 (the same bits of y), and writes
// the double sums of z and z*z over them to stats[(m * pieces + piece) * 2].
// Q4 (N % 4 == 0, 16-byte aligned partials): thread t takes the quad of
// columns 4t .. 4t + 3 of the block's span, as k_splitk_nchw4 does.
constexpr uint32_t kStatsSpan = 1024;
template <bool Q4>
__global__ void __launch_bounds__(256)
    k_splitk_nchw_stats(const float* __restrict__ part, const float* __restrict__ bias,
                        float* __restrict__ out, uint32_t M, uint32_t N, uint32_t HW,
                        uint32_t splits, uint32_t act, double* __restrict__ stats,
                        uint32_t pieces, FastDiv dHW) {
  __shared__ double sh[4];
  const uint32_t m = blockIdx.y, piece = blockIdx.x;
  const float bv = bias ? bias[m] : 0.f;
  double a0 = 0.0, a1 = 0.0;
  if constexpr (Q4) {
    const uint32_t n0 = piece * kStatsSpan + 4 * threadIdx.x;
    if (n0 < N) {
      const size_t nq = size_t(M) * (N / 4);
      f4 z = sum_splits4(reinterpret_cast<const f4*>(part) + (size_t(m) * N + n0) / 4, nq, splits);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        z[e] = epi_act(z[e] + bv, act);
        a0 += double(z[e]);
        a1 += double(z[e]) * double(z[e]);
      }
      uint32_t b = fdiv(n0, dHW), pix = n0 - b * HW;
      if (pix + 3 < HW) {
        stu(out + (size_t(b) * M + m) * HW + pix, z);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          out[(size_t(b) * M + m) * HW + pix] = z[e];
          if (++pix == HW) {
            pix = 0;
            ++b;
          }
        }
      }
    }
  } else {
#pragma unroll
    for (uint32_t u = 0; u < kStatsSpan / 256; ++u) {
      const uint32_t n = piece * kStatsSpan + u * 256 + threadIdx.x;
      if (n >= N) break;
      const size_t i = size_t(m) * N + n;
      float z = 0.f;
      for (uint32_t k = 0; k < splits; ++k) z += part[size_t(k) * M * N + i];
      z = epi_act(z + bv, act);
      const uint32_t b = fdiv(n, dHW), pix = n - b * HW;
      out[(size_t(b) * M + m) * HW + pix] = z;
      a0 += double(z);
      a1 += double(z) * double(z);
    }
  }
  const double s0 = block_sum256(a0, sh);
  const double s1 = block_sum256(a1, sh);
  if (threadIdx.x == 0) {
    double* d = stats + (size_t(m) * pieces + piece) * 2;
    d[0] = s0;
    d[1] = s1;
  }
}

// Zero-padded copy of a row-major [rows][cols] matrix to row stride ldp.
__global__ void k_pad_cols(const float* __restrict__ in, float* __restrict__ out, uint32_t rows,
                           uint32_t cols, uint32_t ldp) {
  const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= size_t(rows) * ldp) return;
  const uint32_t r = uint32_t(i / ldp), c = uint32_t(i - size_t(r) * ldp);
  out[i] = c < cols ? in[size_t(r) * cols + c] : 0.f;
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
// Operands are read through buffer resources addressed by 32-bit float
// offsets below kOob.
static bool operand_fits(size_t floats, const char* what) {
  if (floats < kOob) return true;
  set_error("%s: operand of %zu floats exceeds the implicit-GEMM limit of %u floats (2 GiB)", what,
            floats, kOob);
  return false;
}

struct TileCfg {
  int MT, NT, KT;
  uint32_t splits;
};

// Tuning overrides: DCE_TUNE_<FWD|DW|DX|GEMM>="MT,NT,KT,splits" replaces the
// heuristic choice for that GEMM family (read on every call).
static bool tune_override(const char* var, TileCfg& c) {
  const char* e = getenv(var);
  if (!e || !*e) return false;
  int a, b, k;
  unsigned sp;
  if (sscanf(e, "%d,%d,%d,%u", &a, &b, &k, &sp) != 4) return false;
  c = TileCfg{a, b, k, sp ? sp : 1u};
  return true;
}

// XCD-contiguous tile order (on unless DCE_XCD=0; read on every call).
static bool xcd_order() {
  const char* e = getenv("DCE_XCD");
  return !(e && *e && atoi(e) == 0);
}

// 128 unless 64 wastes clearly less padding (8 % or more of the extent: the
// 576 taps x channels of a 3x3 conv over 64 channels run 11 % padding MFMA
// work on 128-wide dW tiles, and 64-wide ones measured 7 % faster on the
// 128 x 64 x 56 x 56 conv's dW, 3 % on UNet's 64-channel layers).
static int pick_tile(uint32_t extent) {
  const uint64_t w128 = uint64_t(cdiv(extent, 128)) * 128, w64 = uint64_t(cdiv(extent, 64)) * 64;
  return (w128 * 100 > w64 * 108) ? 64 : 128;
}

// Rows of the output tile (the channel axis): the narrow 16- and 32-row tiles
// for up to 16 / 32 channels, where a 64-row tile would feed the matrix unit
// mostly zero rows.
static int pick_tile_m(uint32_t M) {
  if (M <= 16) return 16;
  if (M <= 32) return 32;
  return pick_tile(M);
}

// Workgroups of one kernel instantiation that fit on a CU at once.
template <class Kern>
static int occupancy(Kern kernel) {
  static std::map<const void*, int> cache;
  const void* key = reinterpret_cast<const void*>(kernel);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, kThreads, 0) != hipSuccess || n < 1)
    n = 1;
  cache[key] = n;
  return n;
}

// Estimated microseconds of one launch plus its split-K finish, used to pick
// the split count.  The W = tiles * splits workgroups are spread evenly over
// the CUs; the busiest CU gets n = ceil(W / CUs) of them and runs them in
// batches of at most `occ` (the kernel's workgroups per CU).  In a batch of r
// workgroups one K tile takes max(kLatencyUs, r * tm), where tm is the K
// tile's MFMA time for a lone workgroup (MT*NT*KT*2 flops at the CU's
// 614 GFLOP/s fp32 matrix peak) and kLatencyUs the latency-bound floor, so a
// short last batch costs less than a full one.  Split partials cost
// 2 * splits * M * N * 4 bytes at kFinishBytesPerUs.  The constants were
// fitted to a sweep of every split count of the AlexNet convolutions on
// MI355X: the choices are within 1 % of the best measured configurations.
constexpr double kCuFlopsPerUs = 614.4e3;
constexpr double kLatencyUs = 2.0;
constexpr double kFinishBytesPerUs = 3.0e6;
static double est_us(uint32_t M, uint32_t N, uint32_t kdim, const TileCfg& c, int occ,
                     bool partials) {
  const uint32_t cus = uint32_t(num_cus());
  const uint32_t tiles = cdiv(M, uint32_t(c.MT)) * cdiv(N, uint32_t(c.NT));
  const uint32_t n = cdiv(tiles * c.splits, cus);
  const uint32_t full = n / uint32_t(occ), rem = n - full * uint32_t(occ);
  const double kps = double(cdiv(kdim, uint32_t(c.KT))) / c.splits;
  const double tm = double(c.MT) * c.NT * c.KT * 2.0 / kCuFlopsPerUs;
  double T = kps * full * std::max(kLatencyUs, occ * tm);
  if (rem > 0) T += kps * std::max(kLatencyUs, rem * tm);
  if (partials) T += 2.0 * c.splits * double(M) * N * 4.0 / kFinishBytesPerUs;
  return T;
}

// Tile / split choice for an M x N output with kdim-long dot products.  The
// tile is 128 or 64 per axis (pick_tile); the split count minimises est_us
// over 1..max_splits with at least 8 K tiles per split.  `occ(cfg)` gives the
// occupancy of the kernel that cfg launches; `dense_out` says the unsplit
// launch writes the final output (no partial buffer).
template <class OccFn>
static TileCfg choose(const char* var, uint32_t M, uint32_t N, uint32_t kdim, uint32_t max_splits,
                      bool dense_out, OccFn&& occ, bool kt16_only = false,
                      bool narrow_ksplit = false, bool narrow32 = false) {
  TileCfg c{pick_tile_m(M), pick_tile(N), 16, 1};
  if (kt16_only && c.MT < 64) c.NT = 128;  // the pixel GEMMs' narrow tiles are 128 or 256 wide
  if (narrow_ksplit && c.MT < 64) {
    // Narrow tiles with the waves splitting K: 64 columns (a wave then holds
    // the whole tile's accumulators; 128 would cost registers and occupancy),
    // or 32 (narrow32) when 64 pads the columns by 8 % more: the 144 and 288
    // taps x channels of 3x3 convs over 16 and 32 channels.
    const uint64_t w64 = uint64_t(cdiv(N, 64)) * 64, w32 = uint64_t(cdiv(N, 32)) * 32;
    c.NT = (narrow32 && w64 * 100 > w32 * 108) ? 32 : 64;
    c.KT = 64;
  }
  const uint32_t ktiles = cdiv(kdim, uint32_t(c.KT));
  if (tune_override(var, c)) {
    if (kt16_only) c.KT = 16;
    c.splits = std::max<uint32_t>(1, std::min<uint32_t>(c.splits, cdiv(kdim, uint32_t(c.KT))));
    return c;
  }
  const uint32_t smax = std::max<uint32_t>(1, std::min(max_splits, ktiles / 8));
  double best = 0;
  uint32_t bestS = 1;
  for (uint32_t sp = 1; sp <= smax; ++sp) {
    TileCfg t = c;
    t.splits = sp;
    const double e = est_us(M, N, kdim, t, occ(t), sp > 1 || !dense_out);
    if (sp == 1 || e < best) {
      best = e;
      bestS = sp;
    }
  }
  c.splits = bestS;
  // A 128 x 256 tile (two workgroups per CU) beats 128 x 128 (four) on the
  // pixel-row GEMMs whose rows fill whole 128-row tiles, that need split K to
  // fill the chip and whose 128 x 256 grid still gives every CU about two
  // workgroups: AlexNet b128 c4 / c5 forward and c5 dX (510 workgroups) 3-5 %
  // faster at the same split count.  Unsplit ones (c3 forward, the 56x56
  // single conv) run as fast or slower on it, and small grids (UNet's 32x32
  // and 16x16 levels: 64-384 workgroups) lose up to half their speed.
  if (kt16_only && c.MT == 128 && c.NT == 128 && M % 128 == 0 && c.splits >= 2 &&
      uint64_t(cdiv(M, 128)) * cdiv(N, 256) * c.splits * 8 >= uint64_t(num_cus()) * 15)
    c.NT = 256;
  if (const char* e = getenv("DCE_TUNE_LOG")) {
    if (*e && *e != '0')
      fprintf(stderr, "[dcengine] %s M=%u N=%u K=%u -> %dx%dx%d splits %u (occupancy %d)\n", var, M,
              N, kdim, c.MT, c.NT, c.KT, c.splits, occ(c));
  }
  return c;
}

// Pixel-row GEMMs (forward, dX) of convolutions with few channels on small
// images: at most 128 output rows, dot products of at most 1152 (128
// channels x 3 x 3) and at most 131072 pixels (UNet-base16 b8 below the
// 256^2 level).  The cost model prices their K tiles at its 2 us latency
// floor and splits them 4-7 ways or runs them on 128-row tiles (M = 96);
// measured, unsplit 32-row tiles over more workgroups are 10-20 % faster
// (UNet levels 1-3: 36-41 -> 31-36 us per layer, M = 96 dX 92 -> 73 us).
// An override through DCE_TUNE_* keeps its tile.
static void narrow_short_k(TileCfg& c, const char* var, uint32_t M, uint32_t N, uint32_t kdim) {
  if (const char* e = getenv(var))
    if (*e) return;
  if (M > 128 || kdim > 1152 || N > 131072) return;
  c = TileCfg{M <= 16 ? 16 : 32, 128, 16, 1};
}

template <int MT, int NT, int KT, class LA, class LB, class EPI>
static bool launch(const typename LA::Params& pa, const typename LB::Params& pb,
                   const typename EPI::Params& pe, uint32_t M, uint32_t N, uint32_t ktiles,
                   uint32_t splits, const char* what) {
  const TileGrid tg{cdiv(M, MT), cdiv(N, NT), xcd_order() ? 1u : 0u};
  const uint32_t nwg = tg.gm * tg.gn * splits;
  hipLaunchKernelGGL((k_igemm<MT, NT, KT, LA, LB, EPI>), dim3(nwg), dim3(kThreads), 0, stream(),
                     pa, pb, pe, tg, ktiles, splits);
  return check_launch(what);
}

// Dispatch a functor over the (MT, NT) tile shapes: 64/128 square-ish tiles at
// two KT depths and the narrow MT = 16/32 tiles at KT = 16 (1 x 4 wave grid)
// or KT = 64 (waves split the K tile).  NARROW32: also 32 columns at KT = 64
// (the conv dW of few output channels over 16 or 32 input channels).
template <bool NARROW32 = false, class F>
static bool tiles_dispatch(const TileCfg& c, F&& f) {
#define DCE_T(a, b, k) \
  if (c.MT == a && c.NT == b && c.KT == k) return f.template run<a, b, k>();
  DCE_T(128, 128, 32) DCE_T(128, 64, 32) DCE_T(64, 128, 32) DCE_T(64, 64, 32)
  DCE_T(256, 128, 16) DCE_T(128, 256, 16)
  DCE_T(128, 128, 16) DCE_T(128, 64, 16) DCE_T(64, 128, 16) DCE_T(64, 64, 16)
  DCE_T(32, 128, 16) DCE_T(32, 64, 16) DCE_T(16, 128, 16) DCE_T(16, 64, 16)
  DCE_T(32, 128, 64) DCE_T(32, 64, 64) DCE_T(16, 128, 64) DCE_T(16, 64, 64)
  if constexpr (NARROW32) {
    DCE_T(32, 32, 64) DCE_T(16, 32, 64)
  }
#undef DCE_T
  set_error("igemm: unsupported tile %dx%dx%d", c.MT, c.NT, c.KT);
  return false;
}

// The KT = 16 shapes of the pixel-row GEMMs (forward, dX): the narrow tiles
// come with 128 or 256 pixel columns.
template <class F>
static bool tiles_dispatch16(const TileCfg& c, F&& f) {
#define DCE_T(a, b) \
  if (c.MT == a && c.NT == b && c.KT == 16) return f.template run<a, b, 16>();
  DCE_T(256, 128) DCE_T(128, 256)
  DCE_T(128, 128) DCE_T(128, 64) DCE_T(64, 128) DCE_T(64, 64)
  DCE_T(32, 256) DCE_T(32, 128) DCE_T(16, 256) DCE_T(16, 128)
#undef DCE_T
  set_error("igemm: unsupported tile %dx%dx%d", c.MT, c.NT, c.KT);
  return false;
}
template <class F>
static int tiles_occ16(const TileCfg& c, const F& f) {
#define DCE_T(a, b) \
  if (c.MT == a && c.NT == b && c.KT == 16) return f.template occ<a, b, 16>(c.splits > 1);
  DCE_T(256, 128) DCE_T(128, 256)
  DCE_T(128, 128) DCE_T(128, 64) DCE_T(64, 128) DCE_T(64, 64)
  DCE_T(32, 256) DCE_T(32, 128) DCE_T(16, 256) DCE_T(16, 128)
#undef DCE_T
  return 1;
}

// Occupancy of the kernel a functor would launch for cfg.
template <bool NARROW32 = false, class F>
static int tiles_occ(const TileCfg& c, const F& f) {
#define DCE_T(a, b, k) \
  if (c.MT == a && c.NT == b && c.KT == k) return f.template occ<a, b, k>(c.splits > 1);
  DCE_T(128, 128, 32) DCE_T(128, 64, 32) DCE_T(64, 128, 32) DCE_T(64, 64, 32)
  DCE_T(256, 128, 16) DCE_T(128, 256, 16)
  DCE_T(128, 128, 16) DCE_T(128, 64, 16) DCE_T(64, 128, 16) DCE_T(64, 64, 16)
  DCE_T(32, 128, 16) DCE_T(32, 64, 16) DCE_T(16, 128, 16) DCE_T(16, 64, 16)
  DCE_T(32, 128, 64) DCE_T(32, 64, 64) DCE_T(16, 128, 64) DCE_T(16, 64, 64)
  if constexpr (NARROW32) {
    DCE_T(32, 32, 64) DCE_T(16, 32, 64)
  }
#undef DCE_T
  return 1;
}

static inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
static inline size_t al64(size_t n) { return (n + 63) & ~size_t(63); }

static bool split_nchw_stats(const float* part, const float* bias, float* out, uint32_t M,
                             uint32_t N, uint32_t HW, uint32_t splits, uint32_t act,
                             double* stats, uint32_t pieces) {
  if (N % 4 == 0 && aligned16(part))
    hipLaunchKernelGGL(k_splitk_nchw_stats<true>, dim3(pieces, M), dim3(256), 0, stream(), part,
                       bias, out, M, N, HW, splits, act, stats, pieces, make_fastdiv(HW));
  else
    hipLaunchKernelGGL(k_splitk_nchw_stats<false>, dim3(pieces, M), dim3(256), 0, stream(), part,
                       bias, out, M, N, HW, splits, act, stats, pieces, make_fastdiv(HW));
  return check_launch("splitk_nchw");
}
static bool split_nchw(const float* part, const float* bias, float* out, uint32_t M, uint32_t N,
                       uint32_t HW, uint32_t splits, uint32_t act) {
  if (N % 4 == 0 && aligned16(part))
    hipLaunchKernelGGL(k_splitk_nchw4, dim3(cdiv(size_t(M) * (N / 4), 256)), dim3(256), 0,
                       stream(), reinterpret_cast<const f4*>(part), bias, out, M, N, HW, splits,
                       act);
  else
    hipLaunchKernelGGL(k_splitk_nchw, dim3(cdiv(size_t(M) * N, 256)), dim3(256), 0, stream(),
                       part, bias, out, M, N, HW, splits, act);
  return check_launch("splitk_nchw");
}

// Deterministic split-K sum of row-major partials into c (n elements).
static bool split_sum(const float* part, float* c, uint32_t n, uint32_t splits) {
  if (n % 4 == 0 && aligned16(part) && aligned16(c))
    hipLaunchKernelGGL(k_splitk_sum4, dim3(cdiv(n / 4, 256u)), dim3(256), 0, stream(),
                       reinterpret_cast<const f4*>(part), reinterpret_cast<f4*>(c), n / 4, splits);
  else
    hipLaunchKernelGGL(k_splitk_sum, dim3(cdiv(n, 256u)), dim3(256), 0, stream(), part, c, n,
                       splits);
  return check_launch("splitk_sum");
}

// ----------------------------------------------------------------- GEMM
template <bool AT, bool BT>
struct GemmRun {
  const float *a, *b;
  float* c;
  uint32_t M, K, N, splits;
  uint32_t lda, ldb, kdA, kdB;  // row strides and K extents as stored (padded)
  float* part;                  // split-K partials (splits > 1)
  // A[m][k]: stored M x K (ROWK) or K x M (KROW); B[n][k]: stored N x K (ROWK) or K x N (KROW).
  template <int MT, int KT>
  using LAt = typename std::conditional<AT, LdDenseKR<MT, KT>, LdDenseRK<MT, KT>>::type;
  template <int NT, int KT>
  using LBt = typename std::conditional<BT, LdDenseRK<NT, KT>, LdDenseKR<NT, KT>>::type;
  template <int MT, int NT, int KT>
  int occ(bool) const {
    return occupancy(k_igemm<MT, NT, KT, LAt<MT, KT>, LBt<NT, KT>, EpiRowMajor>);
  }
  template <int MT, int NT, int KT>
  bool run() {
    using LA = LAt<MT, KT>;
    using LB = LBt<NT, KT>;
    const typename LA::Params pa{a, lda, AT ? lda : M, kdA, (AT ? K : M) * lda};
    const typename LB::Params pb{b, ldb, BT ? N : ldb, kdB, (BT ? N : K) * ldb};
    const uint32_t kt = cdiv(std::max(kdA, kdB), KT);
    const EpiRowMajor::Params pe{c, M, N, N, M * N};
    if (splits > 1) {
      const EpiRowMajor::Params pr{part, M, N, N, M * N};
      return launch<MT, NT, KT, LA, LB, EpiRowMajor>(pa, pb, pr, M, N, kt, splits, "gemm") &&
             split_sum(part, c, M * N, splits);
    }
    return launch<MT, NT, KT, LA, LB, EpiRowMajor>(pa, pb, pe, M, N, kt, 1, "gemm");
  }
};

bool gemm(const float* a, const float* b, float* c, uint32_t M, uint32_t K, uint32_t N,
          uint32_t flags) {
  if (K == 0) return fill_zero(c, size_t(M) * N);
  const bool aT = flags & 1, bT = flags & 2;
  if (!operand_fits(size_t(M) * pad4(K), "gemm") || !operand_fits(size_t(K) * pad4(N), "gemm") ||
      !operand_fits(size_t(pad4(M)) * K, "gemm") || !operand_fits(size_t(N) * pad4(K), "gemm"))
    return false;
  // The dense loaders read whole quads along each operand's contiguous axis:
  // a stride that is not a multiple of 4 (or an unaligned base) gets a
  // zero-padded copy.
  const uint32_t aRows = aT ? K : M, aCols = aT ? M : K;
  const uint32_t bRows = bT ? N : K, bCols = bT ? K : N;
  const bool padA = (aCols % 4) || !aligned16(a), padB = (bCols % 4) || !aligned16(b);
  auto gemm_occ = [&](const TileCfg& t) {
    if (!aT && !bT) return tiles_occ(t, GemmRun<false, false>{});
    if (!aT && bT) return tiles_occ(t, GemmRun<false, true>{});
    if (aT && !bT) return tiles_occ(t, GemmRun<true, false>{});
    return tiles_occ(t, GemmRun<true, true>{});
  };
  TileCfg cfg = choose("DCE_TUNE_GEMM", M, N, pad4(K), 16, true, gemm_occ);
  // A grid that leaves CUs idle (small GEMMs such as AlexNet's fc3) runs
  // faster on 64 x 64 tiles 32 deep, at split counts that fill the chip:
  // fc3 forward 34 -> 22 us, its dA 29 -> 24 us in a sweep of every tile
  // and split count on MI355X.
  const uint32_t cus = uint32_t(num_cus());
  auto wgs = [&](const TileCfg& t) {
    return cdiv(M, uint32_t(t.MT)) * cdiv(N, uint32_t(t.NT)) * t.splits;
  };
  if (!getenv("DCE_TUNE_GEMM") && wgs(cfg) < cus && M >= 64 && N >= 64) {
    const uint32_t kt32 = cdiv(pad4(K), 32u);
    TileCfg alt{64, 64, 32, 1};
    const uint32_t t64 = cdiv(M, 64u) * cdiv(N, 64u);
    // The fewest splits that fill every CU, keeping at least 8 K tiles each.
    while (t64 * alt.splits < cus && alt.splits < 16 && kt32 / (alt.splits + 1) >= 8) alt.splits++;
    if (wgs(alt) > wgs(cfg)) cfg = alt;
  }
  // Skinny products with long dot products (a linear layer's forward and
  // input gradient at batch 128): 64 x 64 tiles 32 deep over about 1024
  // workgroups beat the 128 x 128 split-K choice (AlexNet fc1 forward 104 ->
  // 97 us, fc2 forward 56 -> 50 us, fc2 input gradient 53 -> 49 us in a sweep
  // of tiles and split counts on MI355X; wider grids, such as fc1's input
  // gradient with 288 such tiles, keep the model's choice).
  if (!getenv("DCE_TUNE_GEMM") && M <= 128 && pad4(K) >= 4096) {
    const uint32_t t64 = cdiv(M, 64u) * cdiv(N, 64u), kt32 = cdiv(pad4(K), 32u);
    if (t64 >= 64 && t64 <= 256) {
      TileCfg alt{64, 64, 32, std::max(1u, std::min(16u, 1024u / t64))};
      while (alt.splits > 1 && kt32 / alt.splits < 8) alt.splits--;
      cfg = alt;
    }
  }
  const size_t nA = padA ? al64(size_t(aRows) * pad4(aCols)) : 0;
  const size_t nB = padB ? al64(size_t(bRows) * pad4(bCols)) : 0;
  const size_t nP = cfg.splits > 1 ? size_t(cfg.splits) * M * N : 0;
  float* ws = (nA + nB + nP) ? workspace(nA + nB + nP) : nullptr;
  if ((nA + nB + nP) && !ws) return false;
  const float* ap = a;
  const float* bp = b;
  if (padA) {
    hipLaunchKernelGGL(k_pad_cols, dim3(cdiv(nA, 256)), dim3(256), 0, stream(), a, ws, aRows,
                       aCols, pad4(aCols));
    if (!check_launch("gemm_pad")) return false;
    ap = ws;
  }
  if (padB) {
    hipLaunchKernelGGL(k_pad_cols, dim3(cdiv(nB, 256)), dim3(256), 0, stream(), b, ws + nA,
                       bRows, bCols, pad4(bCols));
    if (!check_launch("gemm_pad")) return false;
    bp = ws + nA;
  }
  float* part = cfg.splits > 1 ? ws + nA + nB : nullptr;
  const uint32_t lda = pad4(aCols), ldb = pad4(bCols);
  // K extents: a ROWK operand's k axis is its padded row (zeros past K); a
  // KROW operand's k axis is its row count K.
  const uint32_t kdA = aT ? K : lda, kdB = bT ? ldb : K;
  bool ok;
  {
    ProfScope prof("gemm", 2.0 * M * N * double(K),
                   4.0 * (double(M) * K + double(K) * N + double(M) * N));
    if (!aT && !bT)
      ok = tiles_dispatch(cfg, GemmRun<false, false>{ap, bp, c, M, K, N, cfg.splits, lda, ldb, kdA, kdB, part});
    else if (!aT && bT)
      ok = tiles_dispatch(cfg, GemmRun<false, true>{ap, bp, c, M, K, N, cfg.splits, lda, ldb, kdA, kdB, part});
    else if (aT && !bT)
      ok = tiles_dispatch(cfg, GemmRun<true, false>{ap, bp, c, M, K, N, cfg.splits, lda, ldb, kdA, kdB, part});
    else
      ok = tiles_dispatch(cfg, GemmRun<true, true>{ap, bp, c, M, K, N, cfg.splits, lda, ldb, kdA, kdB, part});
  }
  return ok;
}

// ----------------------------------------------------------- NHWC copies
size_t nhwc_floats(uint32_t B, uint32_t C, uint32_t H, uint32_t W) {
  return size_t(B) * H * W * pad4(C);
}

// Bias-gradient partial rows per channel of the transpose pass (the pixel
// blocks of every plane): 128-pixel blocks for up to 16 channels, else 64.
static uint32_t to_nhwc_rows(uint32_t B, uint32_t Cp, uint32_t HW) {
  return B * (Cp <= 16 ? cdiv(HW, 128) : cdiv(HW, 64));
}

static bool to_nhwc_masked(const float* in, const float* y, float* out, float* dbPart,
                           uint32_t B, uint32_t C, uint32_t HW, uint32_t* npbOut,
                           const WPerm& pw = WPerm{}) {
  const uint32_t Cp = pad4(C);
  // Family "conv_grad_nhwc": the masked dy -> G pass of the conv backward
  // (reads dy and y, writes G); "nhwc": a plain copy of an activation.
  ProfScope prof(y ? "conv_grad_nhwc" : "nhwc", 0,
                 4.0 * double(B) * HW * ((y ? 2.0 : 1.0) * C + Cp));
  if (Cp <= 8 && !y && !dbPart) {
    const uint32_t npix = B * HW;
    hipLaunchKernelGGL(k_to_nhwc_small, dim3(cdiv(npix, 256)), dim3(256), 0, stream(), in, out, C,
                       HW, Cp, npix, make_fastdiv(HW));
    return check_launch("to_nhwc") && (!pw.w || permute_w(pw));
  }
  if (Cp <= 16) {
    const uint32_t npb = cdiv(HW, 128), nMain = npb * B;
    if (npbOut) *npbOut = npb;
    hipLaunchKernelGGL(k_to_nhwc<16>, dim3(nMain + pw.blocks()), dim3(256), 0, stream(), in, y,
                       out, dbPart, C, HW, Cp, npb, 1u, B, nMain, pw);
  } else {
    const uint32_t npb = cdiv(HW, 64);
    if (npbOut) *npbOut = npb;
    const uint32_t ncb = cdiv(Cp, 32), nMain = npb * ncb * B;
    hipLaunchKernelGGL(k_to_nhwc<32>, dim3(nMain + pw.blocks()), dim3(256), 0, stream(), in, y,
                       out, dbPart, C, HW, Cp, npb, ncb, B, nMain, pw);
  }
  return check_launch("to_nhwc");
}

uint32_t bn_dx_g_rows(uint32_t B, uint32_t C, uint32_t HW) { return to_nhwc_rows(B, pad4(C), HW); }

bool bn_dx_g(const float* x, const float* dy, const float* mean, const float* var,
             const float* gamma, const float* dg, const float* db, float eps, float* dx,
             float* g, float* dbPart, uint32_t B, uint32_t C, uint32_t HW) {
  const uint32_t Cp = pad4(C);
  if (uint64_t(B) * C * HW >= kOob || uint64_t(B) * HW * Cp >= kOob) return false;
  ProfScope prof("bn_bwd_dx", 0, 4.0 * double(B) * HW * (3.0 * C + Cp));
  const BnDxArgs bn{mean, var, gamma, dg, db, dx, eps, float(uint64_t(B) * HW)};
  // The same blocks (and bias partials) as the conv backward's transpose pass.
  if (Cp <= 16) {
    const uint32_t npb = cdiv(HW, 128), nMain = npb * B;
    hipLaunchKernelGGL((k_to_nhwc<16, true>), dim3(nMain), dim3(256), 0, stream(), dy, x, g,
                       dbPart, C, HW, Cp, npb, 1u, B, nMain, WPerm{}, bn);
  } else {
    const uint32_t npb = cdiv(HW, 64), ncb = cdiv(Cp, 32), nMain = npb * ncb * B;
    hipLaunchKernelGGL((k_to_nhwc<32, true>), dim3(nMain), dim3(256), 0, stream(), dy, x, g,
                       dbPart, C, HW, Cp, npb, ncb, B, nMain, WPerm{}, bn);
  }
  return check_launch("batchnorm_backward_dx");
}

bool to_nhwc(const float* x, float* out, uint32_t B, uint32_t C, uint32_t H, uint32_t W) {
  return to_nhwc_masked(x, nullptr, out, nullptr, B, C, H * W, nullptr);
}

// Channel-packed, zero-padded copy (fewer than four channels): out[((b*Hp +
// h)*Wp + w)*C + c] = x[b][c][h - p][w - p], zero in the border.  A thread
// takes 4 consecutive padded pixels of one row: one 16-byte load per channel
// (4-byte aligned: unaligned access is on) where the 4 source columns lie in
// the image, else element loads, and C 16-byte stores (the 4*C outputs are
// contiguous and 16-byte aligned when Wp % 4 == 0; otherwise element stores).
template <int C>
__global__ void k_to_pk(const float* __restrict__ x, float* __restrict__ out, uint32_t H,
                        uint32_t W, uint32_t p, uint32_t Hp, uint32_t Wp, uint32_t WQ, uint32_t nq,
                        FastDiv dWQ, FastDiv dHp) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= nq) return;
  const uint32_t t = fdiv(i, dWQ), wq = i - t * WQ;  // t = b * Hp + h
  const uint32_t b = fdiv(t, dHp), h = t - b * Hp;
  const uint32_t w0 = 4 * wq, ih = h - p;  // ih wraps when in the border
  const int iw0 = int(w0) - int(p);
  const bool rowin = ih < H;
  const bool fullin = rowin && iw0 >= 0 && iw0 + 4 <= int(W);
  float o[4 * C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const float* src = x + ((size_t(b) * C + c) * H + (rowin ? ih : 0)) * W;
    f4 q;
    if (fullin) {
      q = ldu<f4>(src + iw0);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int iw = iw0 + e;
        q[e] = (rowin && iw >= 0 && iw < int(W)) ? src[iw] : 0.f;
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e * C + c] = q[e];
  }
  float* dst = out + (size_t(t) * Wp + w0) * C;
  if (Wp % 4 == 0) {
#pragma unroll
    for (int k = 0; k < C; ++k) *reinterpret_cast<f4*>(dst + 4 * k) = f4{o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]};
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (w0 + e < Wp) {
#pragma unroll
        for (int c = 0; c < C; ++c) dst[e * C + c] = o[e * C + c];
      }
  }
}

// Stride-phase copy (see PsParams): thread (b, r, c, column quad cq) reads
// the 4*S consecutive source elements of padded row r from column 4*cq*S - p
// (16-byte loads at 4-byte alignment where they lie in the image, element
// loads at its edges) and stores one 16-byte quad per phase.
template <int S>
__global__ void __launch_bounds__(256)
    k_to_ps(const float* __restrict__ x, float* __restrict__ out, uint32_t C, uint32_t H,
            uint32_t W, uint32_t p, uint32_t Hp, uint32_t Ncol, uint32_t nq, FastDiv dNQ,
            FastDiv dC, FastDiv dHp) {
  const uint32_t i = xcd_block_id() * 256 + threadIdx.x;  // neighbouring rows share an L2
  if (i >= nq) return;
  const uint32_t NQ = dNQ.d;
  const uint32_t t = fdiv(i, dNQ), cq = i - t * NQ;     // t = (b*Hp + r)*C + c
  const uint32_t u = fdiv(t, dC), c = t - u * C;        // u = b*Hp + r
  const uint32_t b = fdiv(u, dHp), r = u - b * Hp;
  const uint32_t ih = r - p;                            // wraps in the border
  const int iw0 = int(4 * cq * S) - int(p);
  const bool rowin = ih < H;
  const float* src = x + ((size_t(b) * C + c) * H + (rowin ? ih : 0)) * W;
  float v[4 * S];
  if (rowin && iw0 >= 0 && iw0 + 4 * S <= int(W)) {
#pragma unroll
    for (int q = 0; q < S; ++q) {
      const f4 a = ldu<f4>(src + iw0 + 4 * q);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * q + e] = a[e];
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4 * S; ++j) {
      const int iw = iw0 + j;
      v[j] = (rowin && iw >= 0 && iw < int(W)) ? src[iw] : 0.f;
    }
  }
  float* dst = out + size_t(t) * S * Ncol + 4 * cq;
#pragma unroll
  for (int ph = 0; ph < S; ++ph)
    *reinterpret_cast<f4*>(dst + ph * Ncol) = f4{v[ph], v[S + ph], v[2 * S + ph], v[3 * S + ph]};
}

// Masked gradient on the padded pixel grid for the stride-phase dW GEMM:
// G_pad[b][oc][oh][ow] = dy masked by y (y <= 0 -> 0; a NaN y keeps it) for
// ow < OW, 0 for OW <= ow < OWp.  Block = one chunk of up to kMaskChunk
// padded elements of one (b, oc) plane, four 16-byte quads per thread (all
// loaded before any is stored); dbPart[oc][b*nchunk + chunk] = the block's
// sum of the masked values (thread, wave, then wave order).
constexpr uint32_t kMaskChunk = 4096;
__global__ void __launch_bounds__(256)
    k_mask_pad(const float* __restrict__ dy, const float* __restrict__ y, float* __restrict__ g,
               float* __restrict__ dbPart, uint32_t OC, uint32_t OH, uint32_t OW, uint32_t OWp,
               uint32_t nchunk, uint32_t nB, FastDiv dChunk, FastDiv dOWp) {
  __shared__ float sh[4];
  // XCD-contiguous numbering: neighbouring chunks share the cache lines of
  // rows of odd length, and then share an L2.
  const uint32_t id = xcd_block_id();
  const uint32_t plane = fdiv(id, dChunk), chunk = id - plane * nchunk;
  const uint32_t OHWp = OH * OWp;
  const float* dyp = dy + size_t(plane) * OH * OW;
  const float* yp = y ? y + size_t(plane) * OH * OW : nullptr;
  // Every quad is one 16-byte load (4-byte aligned; unaligned access is on),
  // issued back to back with no branch between them: a quad that would run
  // past its row (or a thread past the plane) loads the 4 elements ending at
  // the row's last one (at the plane's start) and shifts them into place,
  // zero-filling.  Rows of fewer than 4 elements take element loads.
  f4 v[4], m[4];
  uint32_t e[4];
  if (OW >= 4) {
    uint32_t shift[4], src[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      e[j] = chunk * kMaskChunk + 4 * (threadIdx.x + 256 * j);
      const uint32_t ej = e[j] < OHWp ? e[j] : 0u;
      const uint32_t oh = fdiv(ej, dOWp), ow = ej - oh * OWp;
      shift[j] = ow + 4 <= OW ? 0u : ow + 4 - OW;  // 1..3 for a row's last quad
      src[j] = oh * OW + ow - shift[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = ldu<f4>(dyp + src[j]);
      m[j] = yp ? ldu<f4>(yp + src[j]) : f4{1.f, 1.f, 1.f, 1.f};
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t d = shift[j];
      const f4 a = v[j], b = m[j];
      v[j] = f4{d == 0 ? a[0] : d == 1 ? a[1] : d == 2 ? a[2] : a[3],
                d == 0 ? a[1] : d == 1 ? a[2] : d == 2 ? a[3] : 0.f,
                d == 0 ? a[2] : d == 1 ? a[3] : 0.f, d == 0 ? a[3] : 0.f};
      m[j] = f4{d == 0 ? b[0] : d == 1 ? b[1] : d == 2 ? b[2] : b[3],
                d == 0 ? b[1] : d == 1 ? b[2] : d == 2 ? b[3] : 1.f,
                d == 0 ? b[2] : d == 1 ? b[3] : 1.f, d == 0 ? b[3] : 1.f};
      if (e[j] >= OHWp) v[j] = f4{0.f, 0.f, 0.f, 0.f};
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      e[j] = chunk * kMaskChunk + 4 * (threadIdx.x + 256 * j);
      v[j] = m[j] = f4{0.f, 0.f, 0.f, 0.f};
      if (e[j] >= OHWp) continue;
      const uint32_t oh = fdiv(e[j], dOWp), ow = e[j] - oh * OWp;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[j][q] = ow + q < OW ? dyp[oh * OW + ow + q] : 0.f;
        m[j][q] = (yp && ow + q < OW) ? yp[oh * OW + ow + q] : 1.f;
      }
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int q = 0; q < 4; ++q) v[j][q] = m[j][q] <= 0.f ? 0.f : v[j][q];
    if (e[j] < OHWp) *reinterpret_cast<f4*>(g + size_t(plane) * OHWp + e[j]) = v[j];
    sum += (v[j][0] + v[j][1]) + (v[j][2] + v[j][3]);
  }
  if (dbPart == nullptr) return;
  sum = wave_reduce(sum);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = sum;
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t b = plane / OC, oc = plane - b * OC;
    dbPart[size_t(oc) * nB * nchunk + size_t(b) * nchunk + chunk] = (sh[0] + sh[1]) + (sh[2] + sh[3]);
  }
}

// Layout of the conv input copy: channel-innermost (C >= 4), stride-phase
// (C < 4, stride <= 4) or channel-packed (C < 4, larger strides).
bool ps_x(const ConvGeom& g) { return g.C < 4 && g.s <= 4; }
// Pointwise convolutions (1 x 1, stride 1, no padding, planes of a multiple
// of 4 pixels, at least 4 channels) read x, dy and write y, dx in NCHW: the
// GEMMs take the planes as they are, with no channel-innermost copy.
bool pw_x(const ConvGeom& g) {
  return g.k == 1 && g.s == 1 && g.p == 0 && (g.H * g.W) % 4 == 0 && g.C >= 4;
}
bool packed_x(const ConvGeom& g) { return g.C < 4 && g.s > 4; }

struct PsGeom {
  uint32_t Hp, OWp, OHWp, Ncol, RS;
  size_t floats;
};
static PsGeom ps_geom(const ConvGeom& g) {
  PsGeom q;
  q.Hp = g.H + 2 * g.p;
  q.OWp = pad4(g.OW);
  q.OHWp = g.OH * q.OWp;
  // Columns: the padded image, and every quad a padded output row's taps
  // read (up to OWp - 1 + (k - 1) / S).
  const uint32_t cols = std::max(cdiv(g.W + 2 * g.p, g.s), q.OWp + (g.k - 1) / g.s);
  q.Ncol = pad4(cols);
  q.RS = g.C * g.s * q.Ncol;
  q.floats = size_t(g.B) * q.Hp * q.RS;
  return q;
}

size_t xcopy_floats(const ConvGeom& g) {
  if (pw_x(g)) return 4;  // no copy: a placeholder handle
  if (ps_x(g)) return ps_geom(g).floats;
  if (!packed_x(g)) return nhwc_floats(g.B, g.C, g.H, g.W);
  return size_t(g.B) * (g.H + 2 * g.p) * (g.W + 2 * g.p) * g.C;
}

// Floats of the copy of x the general conv path builds (a pointwise layer
// that takes that path, for its ReLU mask, needs the NHWC copy its forward
// did not keep).
static size_t xbuild_floats(const ConvGeom& g) {
  return pw_x(g) ? nhwc_floats(g.B, g.C, g.H, g.W) : xcopy_floats(g);
}

uint32_t xcopy_tag(const ConvGeom& g) {
  if (pw_x(g)) return 0x40000u;
  if (ps_x(g)) return 0x20000u + g.p + (g.s << 8) + (g.k << 12);
  return packed_x(g) ? 0x10000u + g.p : pad4(g.C);
}

static bool to_ps(const float* x, float* out, const ConvGeom& g) {
  const PsGeom q = ps_geom(g);
  const uint32_t NQ = q.Ncol / 4, nq = g.B * q.Hp * g.C * NQ;
  ProfScope prof("nhwc", 0, 4.0 * (double(g.B) * g.C * g.H * g.W + double(q.floats)));
  const dim3 grid(cdiv(nq, 256));
  const FastDiv fNQ = make_fastdiv(NQ), fC = make_fastdiv(g.C), fHp = make_fastdiv(q.Hp);
#define DCE_PS(S_)                                                                            \
  if (g.s == S_)                                                                              \
    hipLaunchKernelGGL(k_to_ps<S_>, grid, dim3(256), 0, stream(), x, out, g.C, g.H, g.W, g.p, \
                       q.Hp, q.Ncol, nq, fNQ, fC, fHp);
  DCE_PS(1) DCE_PS(2) DCE_PS(3) DCE_PS(4)
#undef DCE_PS
  return check_launch("to_ps");
}

static PsParams ps_params(const float* src, const ConvGeom& g) {
  const PsGeom q = ps_geom(g);
  const uint32_t KK = g.k * g.k;
  return PsParams{src, q.RS, q.Hp, g.s, q.Ncol, g.C, g.k, KK, g.C * KK, q.OWp, q.OHWp,
                  g.B * q.OHWp, uint32_t(q.floats), make_fastdiv(q.OHWp), make_fastdiv(q.OWp),
                  make_fastdiv(KK), make_fastdiv(g.k), make_fastdiv(g.s)};
}

// G_pad (and, with dbPart, the bias-gradient partials: OC rows of
// B * nchunk); returns nchunk.
static uint32_t mask_pad(const float* dy, const float* y, float* gp, float* dbPart,
                         const ConvGeom& g, bool* ok) {
  const PsGeom q = ps_geom(g);
  const uint32_t nchunk = cdiv(q.OHWp, kMaskChunk), planes = g.B * g.OC;
  ProfScope prof("conv_grad_nhwc", 0, 4.0 * (2.0 * g.B * g.OC * g.OH * g.OW + double(planes) * q.OHWp));
  hipLaunchKernelGGL(k_mask_pad, dim3(planes * nchunk), dim3(256), 0, stream(), dy, y, gp, dbPart,
                     g.OC, g.OH, g.OW, q.OWp, nchunk, g.B, make_fastdiv(nchunk),
                     make_fastdiv(q.OWp));
  *ok = check_launch("mask_pad");
  return nchunk;
}

static bool to_pk(const float* x, float* out, const ConvGeom& g) {
  const uint32_t Hp = g.H + 2 * g.p, Wp = g.W + 2 * g.p, npix = g.B * Hp * Wp;
  const uint32_t WQ = cdiv(Wp, 4), nq = g.B * Hp * WQ;
  ProfScope prof("nhwc", 0, 4.0 * (double(g.B) * g.C * g.H * g.W + double(npix) * g.C));
  const dim3 grid(cdiv(nq, 256));
  const FastDiv fWQ = make_fastdiv(WQ), fHp = make_fastdiv(Hp);
  if (g.C == 1)
    hipLaunchKernelGGL(k_to_pk<1>, grid, dim3(256), 0, stream(), x, out, g.H, g.W, g.p, Hp, Wp, WQ,
                       nq, fWQ, fHp);
  else if (g.C == 2)
    hipLaunchKernelGGL(k_to_pk<2>, grid, dim3(256), 0, stream(), x, out, g.H, g.W, g.p, Hp, Wp, WQ,
                       nq, fWQ, fHp);
  else
    hipLaunchKernelGGL(k_to_pk<3>, grid, dim3(256), 0, stream(), x, out, g.H, g.W, g.p, Hp, Wp, WQ,
                       nq, fWQ, fHp);
  return check_launch("to_pk");
}

static PkParams pk_params(const float* src, const ConvGeom& g) {
  const uint32_t Hp = g.H + 2 * g.p, Wp = g.W + 2 * g.p, OHW = g.OH * g.OW, kC = g.k * g.C;
  return PkParams{src, Wp * g.C, Hp * Wp * g.C, g.C, g.k, g.s, kC, g.k * kC, g.OW, OHW,
                  g.B * OHW, uint32_t(xcopy_floats(g)), make_fastdiv(OHW), make_fastdiv(g.OW),
                  make_fastdiv(kC)};
}

// ----------------------------------------------------------- conv forward
// Output pixels as GEMM columns: split-K partials go to a row-major [M][N]
// workspace and k_splitk_nchw finishes (bias, activation, NCHW scatter).
// K order: blocked when the padded channel count is a multiple of kCB (no
// extra padding then), flat otherwise.
static inline bool blocked_k(uint32_t Cp) { return Cp % kCB == 0; }

// Run F<S1, BLK> for the runtime (stride == 1, blocked) pair.
template <template <bool, bool> class F, class... A>
static bool conv_variant(bool s1, bool blk, const TileCfg& c, A&&... a) {
  if (s1 && blk) return tiles_dispatch16(c, F<true, true>{a...});
  if (s1) return tiles_dispatch16(c, F<true, false>{a...});
  if (blk) return tiles_dispatch16(c, F<false, true>{a...});
  return tiles_dispatch16(c, F<false, false>{a...});
}
template <template <bool, bool> class F>
static int conv_variant_occ(bool s1, bool blk, const TileCfg& c) {
  if (s1 && blk) return tiles_occ16(c, F<true, true>{});
  if (s1) return tiles_occ16(c, F<true, false>{});
  if (blk) return tiles_occ16(c, F<false, true>{});
  return tiles_occ16(c, F<false, false>{});
}

template <bool S1, bool BLK>
struct FwdRun {
  const float* wp;
  const float* xn;
  const float* bias;
  float* y;
  float* part;
  ConvGeom g;
  uint32_t act, splits;
  double* stats;  // stride 1: BN statistics of y (pieces as stats_buffer sets them)
  uint32_t pieces;
  template <int MT, int NT, int KT>
  int occ(bool split) const {
    using LA = LdDenseRK<MT, KT>;
    using LB = LdPixRK<NT, KT, true, S1, BLK>;
    return split ? occupancy(k_igemm<MT, NT, KT, LA, LB, EpiRowMajor>)
                 : occupancy(k_igemm<MT, NT, KT, LA, LB, EpiNCHW>);
  }
  template <int MT, int NT, int KT>
  bool run() {
    const uint32_t Cp = pad4(g.C), KK = g.k * g.k, kdim = KK * Cp;
    const uint32_t OHW = g.OH * g.OW, N = g.B * OHW;
    using LA = LdDenseRK<MT, KT>;
    using LB = LdPixRK<NT, KT, true, S1, BLK>;
    const typename LA::Params pa{wp, kdim, g.OC, kdim, g.OC * kdim};
    const typename LB::Params pb{xn, g.H, g.W, Cp, g.k, g.s, g.p, g.OW, OHW, N, kdim,
                                 g.B * g.H * g.W * Cp, make_fastdiv(OHW), make_fastdiv(g.OW),
                                 make_fastdiv(BLK ? KK : Cp), make_fastdiv(g.k)};
    const uint32_t kt = cdiv(kdim, KT);
    const EpiNCHW::Params pe{y, bias, g.OC, OHW, N, act, make_fastdiv(OHW)};
    if (splits > 1) {
      const EpiRowMajor::Params pr{part, g.OC, N, N, g.OC * N};
      return launch<MT, NT, KT, LA, LB, EpiRowMajor>(pa, pb, pr, g.OC, N, kt, splits,
                                                    "conv_forward") &&
             (stats ? split_nchw_stats(part, bias, y, g.OC, N, OHW, splits, act, stats, pieces)
                    : split_nchw(part, bias, y, g.OC, N, OHW, splits, act));
    }
    if constexpr (S1) {
      if (stats) {
        const EpiNCHWStats::Params ps{pe, stats, pieces};
        return launch<MT, NT, KT, LA, LB, EpiNCHWStats>(pa, pb, ps, g.OC, N, kt, 1,
                                                        "conv_forward");
      }
    }
    return launch<MT, NT, KT, LA, LB, EpiNCHW>(pa, pb, pe, g.OC, N, kt, 1, "conv_forward");
  }
};

// Forward over the channel-packed copy (C < 4): K runs over the unpadded
// taps (kh, kw, c), filters padded to pad4(KK * C) per row.
struct FwdPkRun {
  const float* wp;
  const float* xp;
  const float* bias;
  float* y;
  float* part;
  ConvGeom g;
  uint32_t act, splits;
  template <int MT, int NT, int KT>
  int occ(bool split) const {
    using LA = LdDenseRK<MT, KT>;
    using LB = LdPkRK<NT, KT>;
    return split ? occupancy(k_igemm<MT, NT, KT, LA, LB, EpiRowMajor>)
                 : occupancy(k_igemm<MT, NT, KT, LA, LB, EpiNCHW>);
  }
  template <int MT, int NT, int KT>
  bool run() {
    const uint32_t kdim = pad4(g.k * g.k * g.C);
    const uint32_t OHW = g.OH * g.OW, N = g.B * OHW;
    using LA = LdDenseRK<MT, KT>;
    using LB = LdPkRK<NT, KT>;
    const typename LA::Params pa{wp, kdim, g.OC, kdim, g.OC * kdim};
    const PkParams pb = pk_params(xp, g);
    const uint32_t kt = cdiv(kdim, KT);
    const EpiNCHW::Params pe{y, bias, g.OC, OHW, N, act, make_fastdiv(OHW)};
    if (splits > 1) {
      const EpiRowMajor::Params pr{part, g.OC, N, N, g.OC * N};
      return launch<MT, NT, KT, LA, LB, EpiRowMajor>(pa, pb, pr, g.OC, N, kt, splits,
                                                    "conv_forward") &&
             split_nchw(part, bias, y, g.OC, N, OHW, splits, act);
    }
    return launch<MT, NT, KT, LA, LB, EpiNCHW>(pa, pb, pe, g.OC, N, kt, 1, "conv_forward");
  }
};

// Forward over the stride-phase copy (C < 4, stride <= 4): K runs over the
// taps (c, kh, kw), the filters' own order (rows padded to pad4(C*KK)); the
// columns are the padded pixel grid, written through EpiNCHWPad (no split).
struct FwdPsRun {
  const float* wp;
  const float* xs;
  const float* bias;
  float* y;
  ConvGeom g;
  uint32_t act;
  template <int MT, int NT, int KT>
  int occ(bool) const {
    return occupancy(k_igemm<MT, NT, KT, LdDenseRK<MT, KT>, LdPsKR<NT, KT>, EpiNCHWPad>);
  }
  template <int MT, int NT, int KT>
  bool run() {
    const uint32_t kdim = pad4(g.C * g.k * g.k);
    using LA = LdDenseRK<MT, KT>;
    using LB = LdPsKR<NT, KT>;
    const typename LA::Params pa{wp, kdim, g.OC, kdim, g.OC * kdim};
    const PsParams pb = ps_params(xs, g);
    const EpiNCHWPad::Params pe{y, bias, g.OC, g.OH * g.OW, g.OW, pb.OWp, pb.OHWp, pb.npix, act,
                                pb.dOHWp, pb.dOWp};
    return launch<MT, NT, KT, LA, LB, EpiNCHWPad>(pa, pb, pe, g.OC, pb.npix, cdiv(kdim, KT), 1,
                                                  "conv_forward");
  }
};

static bool conv_forward_ps(const float* x, float* keep, const float* w, const float* bias,
                            float* y, const ConvGeom& g, uint32_t act) {
  const PsGeom q = ps_geom(g);
  const uint32_t taps = g.C * g.k * g.k, kdim = pad4(taps), N = g.B * q.OHWp;
  if (!operand_fits(q.floats, "conv_forward") || !operand_fits(size_t(g.OC) * kdim, "conv_forward"))
    return false;
  TileCfg cfg = choose("DCE_TUNE_FWD", g.OC, N, kdim, 1, true,
                       [&](const TileCfg& t) { return tiles_occ16(t, FwdPsRun{}); }, true);
  cfg.splits = 1;  // the padded-grid epilogue writes the output directly
  const size_t nw = al64(size_t(g.OC) * kdim);
  float* ws = workspace(nw + (keep ? 0 : al64(q.floats)));
  if (!ws) return false;
  float* xs = keep ? keep : ws + nw;
  if (!to_ps(x, xs, g)) return false;
  hipLaunchKernelGGL(k_pad_cols, dim3(cdiv(nw, 256)), dim3(256), 0, stream(), w, ws, g.OC, taps,
                     kdim);
  if (!check_launch("pad_w")) return false;
  ProfScope prof("conv_fwd", 2.0 * g.OC * taps * double(g.B) * g.OH * g.OW,
                 4.0 * (double(g.B) * g.C * g.H * g.W + double(g.B) * g.OC * g.OH * g.OW));
  return tiles_dispatch16(cfg, FwdPsRun{ws, xs, bias, y, g, act});
}

// Pointwise forward: y[oc][n] = sum_c w[oc][c] x[c][n] over the pixels n =
// b*HW + pix of NCHW x, filters padded to pad4(C) per row.
struct FwdPwRun {
  const float* wp;
  const float* x;
  const float* bias;
  float* y;
  float* part;
  ConvGeom g;
  uint32_t act, splits;
  double* stats;  // BN statistics of y (pieces as stats_buffer sets them)
  uint32_t pieces;
  template <int MT, int NT, int KT>
  int occ(bool split) const {
    using LA = LdDenseRK<MT, KT>;
    using LB = LdNchwKR<NT, KT>;
    return split ? occupancy(k_igemm<MT, NT, KT, LA, LB, EpiRowMajor>)
                 : occupancy(k_igemm<MT, NT, KT, LA, LB, EpiNCHW>);
  }
  template <int MT, int NT, int KT>
  bool run() {
    const uint32_t Cp = pad4(g.C), HW = g.H * g.W, N = g.B * HW;
    using LA = LdDenseRK<MT, KT>;
    using LB = LdNchwKR<NT, KT>;
    const typename LA::Params pa{wp, Cp, g.OC, Cp, g.OC * Cp};
    const NchwKRParams pb{x, g.C, HW, N, g.B * g.C * HW, make_fastdiv(HW)};
    const uint32_t kt = cdiv(Cp, KT);
    const EpiNCHW::Params pe{y, bias, g.OC, HW, N, act, make_fastdiv(HW)};
    if (splits > 1) {
      const EpiRowMajor::Params pr{part, g.OC, N, N, g.OC * N};
      return launch<MT, NT, KT, LA, LB, EpiRowMajor>(pa, pb, pr, g.OC, N, kt, splits,
                                                    "conv_forward") &&
             (stats ? split_nchw_stats(part, bias, y, g.OC, N, HW, splits, act, stats, pieces)
                    : split_nchw(part, bias, y, g.OC, N, HW, splits, act));
    }
    if (stats) {
      const EpiNCHWStats::Params ps{pe, stats, pieces};
      return launch<MT, NT, KT, LA, LB, EpiNCHWStats>(pa, pb, ps, g.OC, N, kt, 1, "conv_forward");
    }
    return launch<MT, NT, KT, LA, LB, EpiNCHW>(pa, pb, pe, g.OC, N, kt, 1, "conv_forward");
  }
};

// The buffer for the BN statistics of a conv forward's output when its GEMM
// leaves them (pixel GEMMs at stride 1 and pointwise GEMMs, no activation):
// one piece per column tile, or per kStatsSpan columns of the split-K finish.
static double* stats_buffer(ConvStatsReq* st, const TileCfg& cfg, uint32_t N, uint32_t act,
                            bool able) {
  if (!st || act != 0 || !able) return nullptr;
  const uint32_t pieces = cfg.splits > 1 ? cdiv(N, kStatsSpan) : cdiv(N, cfg.NT);
  double* d = st->get(st->ctx, pieces);
  if (d) st->pieces = pieces;
  return d;
}

// Pointwise products with dot products of at most 32 (expand forward,
// project dX): streaming-bound, one K tile or two per output tile.  For up to
// 160 output rows, unsplit 32-row tiles (rows filled exactly or nearly, more
// workgroups in flight) measured faster than the 64- and 128-row choices
// (MobileNetV2 b64: 96 x 200704 x 24 dX 37.6 -> 26.7 us, 144 x 200704 x 24
// forward and dX 46.2 -> 42.6 and 43.6 -> 39.9 us, 96 x 802816 x 16 forward
// 110.3 -> 107.4 us); at 192 rows (x 50176 x 32) they were no faster (dX)
// or 5 % slower (forward), so the rule stops at 160.  An override through
// DCE_TUNE_* keeps its tile.
static void narrow_pw(TileCfg& c, const char* var, uint32_t M, uint32_t kdim) {
  if (const char* e = getenv(var))
    if (*e) return;
  if (M <= 32 || M > 160 || kdim > 32) return;
  c = TileCfg{32, 128, 16, 1};
}

static bool conv_forward_pw(const float* x, const float* w, const float* bias, float* y,
                            const ConvGeom& g, uint32_t act, ConvStatsReq* st) {
  const uint32_t Cp = pad4(g.C), N = g.B * g.H * g.W;
  if (!operand_fits(size_t(g.B) * g.C * g.H * g.W, "conv_forward")) return false;
  TileCfg cfg = choose(
      "DCE_TUNE_FWD", g.OC, N, Cp, 8, true,
      [&](const TileCfg& t) { return tiles_occ16(t, FwdPwRun{}); }, true);
  narrow_pw(cfg, "DCE_TUNE_FWD", g.OC, Cp);
  // Filters [OC][C] are already the A operand when C % 4 == 0 (16-byte rows).
  const bool wDirect = g.C % 4 == 0 && aligned16(w);
  const size_t nw = wDirect ? 0 : al64(size_t(g.OC) * Cp);
  const size_t nP = cfg.splits > 1 ? size_t(cfg.splits) * g.OC * N : 0;
  float* ws = (nw + nP) ? workspace(nw + nP) : nullptr;
  if ((nw + nP) && !ws) return false;
  if (!wDirect && !permute_w(WPerm{w, ws, g.OC, g.C, 1, Cp, Cp, 0, 0})) return false;
  ProfScope prof("conv_fwd", 2.0 * g.OC * g.C * double(N),
                 4.0 * (double(g.B) * g.C * g.H * g.W + double(g.B) * g.OC * g.OH * g.OW));
  double* stats = stats_buffer(st, cfg, N, act, true);
  return tiles_dispatch16(cfg, FwdPwRun{wDirect ? w : ws, x, bias, y, ws ? ws + nw : nullptr, g,
                                        act, cfg.splits, stats, st ? st->pieces : 0});
}

bool conv_forward(const float* x, float* x_nhwc_keep, const float* w, const float* bias,
                  float* y, const ConvGeom& g, uint32_t act, ConvStatsReq* st) {
  if (st) st->pieces = 0;
  if (pw_x(g)) return conv_forward_pw(x, w, bias, y, g, act, st);
  if (ps_x(g)) return conv_forward_ps(x, x_nhwc_keep, w, bias, y, g, act);
  const bool pk = packed_x(g);
  const uint32_t Cp = pad4(g.C), KK = g.k * g.k, kdim = pk ? pad4(KK * g.C) : KK * Cp;
  const bool blk = !pk && blocked_k(Cp), s1 = g.s == 1;
  const size_t nx = xcopy_floats(g);
  const uint32_t N = g.B * g.OH * g.OW;
  if (!operand_fits(nx, "conv_forward") || !operand_fits(size_t(g.OC) * kdim, "conv_forward"))
    return false;
  TileCfg cfg = choose(
      "DCE_TUNE_FWD", g.OC, N, kdim, 8, true,
      [&](const TileCfg& t) {
        return pk ? tiles_occ16(t, FwdPkRun{}) : conv_variant_occ<FwdRun>(s1, blk, t);
      },
      true);
  if (!pk) narrow_short_k(cfg, "DCE_TUNE_FWD", g.OC, N, kdim);
  const size_t nw = al64(size_t(g.OC) * kdim);
  const size_t nxs = x_nhwc_keep ? 0 : al64(nx);
  const size_t nP = cfg.splits > 1 ? size_t(cfg.splits) * g.OC * N : 0;
  float* ws = workspace(nw + nxs + nP);
  if (!ws) return false;
  float* wp = ws;
  float* xn = x_nhwc_keep ? x_nhwc_keep : ws + nw;
  float* part = ws + nw + nxs;
  // The filter re-layout rides in the NHWC copy's launch.
  const WPerm fwdPerm{w, wp, g.OC, g.C, KK, pk ? g.C : Cp, kdim, 0, blk ? 1 : 0};
  if (pk ? !(to_pk(x, xn, g) && permute_w(fwdPerm))
         : !to_nhwc_masked(x, nullptr, xn, nullptr, g.B, g.C, g.H * g.W, nullptr, fwdPerm))
    return false;
  const double fl = 2.0 * g.OC * g.C * KK * double(g.B) * g.OH * g.OW;
  {
    ProfScope prof("conv_fwd", fl,
                   4.0 * (double(g.B) * g.C * g.H * g.W + double(g.B) * g.OC * g.OH * g.OW));
    double* stats = stats_buffer(st, cfg, N, act, !pk && s1);
    const bool ok =
        pk ? tiles_dispatch16(cfg, FwdPkRun{wp, xn, bias, y, part, g, act, cfg.splits})
           : conv_variant<FwdRun>(s1, blk, cfg, wp, xn, bias, y, part, g, act, cfg.splits,
                                  stats, st ? st->pieces : 0u);
    if (!ok) return false;
  }
  return true;
}

// ----------------------------------------------------------- conv backward
// dW = G (rows oc) x x-taps (rows (kh, kw, c)), both with k = output pixel.
// `trans` swaps the operands (taps as output rows) for layers with fewer taps
// x channels than output channels, so the narrow tiles cover the short axis.
struct DwRun {
  const float* gn;  // G: NHWC, or G_pad for the stride-phase layout
  const float* xn;
  float* part;
  ConvGeom g;
  uint32_t splits;
  bool trans;
  bool pk;  // xn is the channel-packed copy: taps (kh, kw, c) with C unpadded
  bool ps;  // xn is the stride-phase copy, gn G_pad: taps (c, kh, kw), padded pixels
  template <int MT, int NT, int KT>
  int occ(bool) const {
    if (ps)
      return trans ? occupancy(k_igemm<MT, NT, KT, LdPsRK<MT, KT>, LdGPadRK<NT, KT>, EpiRowMajor>)
                   : occupancy(k_igemm<MT, NT, KT, LdGPadRK<MT, KT>, LdPsRK<NT, KT>, EpiRowMajor>);
    if (pk)
      return trans ? occupancy(k_igemm<MT, NT, KT, LdPkKR<MT, KT>, LdGradKR<NT, KT>, EpiRowMajor>)
                   : occupancy(k_igemm<MT, NT, KT, LdGradKR<MT, KT>, LdPkKR<NT, KT>, EpiRowMajor>);
    return trans ? occupancy(k_igemm<MT, NT, KT, LdXTapKR<MT, KT>, LdGradKR<NT, KT>, EpiRowMajor>)
                 : occupancy(k_igemm<MT, NT, KT, LdGradKR<MT, KT>, LdXTapKR<NT, KT>, EpiRowMajor>);
  }
  template <int MT, int NT, int KT, class LX>
  bool go(const typename LX::Params& px, uint32_t N) {
    const uint32_t OCp = pad4(g.OC), npix = g.B * g.OH * g.OW;
    const GradKRParams pg{gn, OCp, npix, npix * OCp};
    const uint32_t zs = 4 * cdiv(size_t(g.OC) * N, 4);  // split stride of the partials
    if (trans) {
      const EpiRowMajor::Params pe{part, N, g.OC, g.OC, zs};
      return launch<MT, NT, KT, LX, LdGradKR<NT, KT>, EpiRowMajor>(
          px, pg, pe, N, g.OC, cdiv(npix, KT), splits, "conv_backward_filter");
    }
    using LB = typename std::conditional<std::is_same<LX, LdPkKR<MT, KT>>::value, LdPkKR<NT, KT>,
                                         LdXTapKR<NT, KT>>::type;
    const EpiRowMajor::Params pe{part, g.OC, N, N, zs};
    return launch<MT, NT, KT, LdGradKR<MT, KT>, LB, EpiRowMajor>(
        pg, px, pe, g.OC, N, cdiv(npix, KT), splits, "conv_backward_filter");
  }
  template <int MT, int NT, int KT>
  bool run_ps() {
    const PsParams px = ps_params(xn, g);
    const GPadParams pg{gn, g.OC, px.OHWp, px.npix, g.B * g.OC * px.OHWp, px.dOHWp};
    const uint32_t N = px.kdim, zs = 4 * cdiv(size_t(g.OC) * N, 4), kt = cdiv(px.npix, KT);
    if (trans) {
      const EpiRowMajor::Params pe{part, N, g.OC, g.OC, zs};
      return launch<MT, NT, KT, LdPsRK<MT, KT>, LdGPadRK<NT, KT>, EpiRowMajor>(
          px, pg, pe, N, g.OC, kt, splits, "conv_backward_filter");
    }
    const EpiRowMajor::Params pe{part, g.OC, N, N, zs};
    return launch<MT, NT, KT, LdGPadRK<MT, KT>, LdPsRK<NT, KT>, EpiRowMajor>(
        pg, px, pe, g.OC, N, kt, splits, "conv_backward_filter");
  }
  template <int MT, int NT, int KT>
  bool run() {
    const uint32_t KK = g.k * g.k, OHW = g.OH * g.OW, npix = g.B * OHW;
    if (ps) return run_ps<MT, NT, KT>();
    if (pk) return go<MT, NT, KT, LdPkKR<MT, KT>>(pk_params(xn, g), KK * g.C);
    const uint32_t Cp = pad4(g.C), N = KK * Cp;
    const XTapParams px{xn, g.H, g.W, Cp, g.k, g.s, g.p, g.OW, OHW, npix, N,
                        g.B * g.H * g.W * Cp, make_fastdiv(OHW), make_fastdiv(g.OW),
                        make_fastdiv(Cp), make_fastdiv(g.k)};
    return go<MT, NT, KT, LdXTapKR<MT, KT>>(px, N);
  }
};

// Fraction of an M x N tile grid's area that is real output.
static double tile_fill(uint32_t M, uint32_t N) {
  const double mt = pick_tile_m(M), nt = pick_tile(N);
  return double(M) * N / (std::ceil(M / mt) * mt * std::ceil(N / nt) * nt);
}

template <bool S1, bool BLK>
struct DxRun {
  const float* wt;
  const float* gn;
  float* dx;
  float* part;
  ConvGeom g;
  uint32_t splits;
  template <int MT, int NT, int KT>
  int occ(bool split) const {
    using LA = LdDenseRK<MT, KT>;
    using LB = LdPixRK<NT, KT, false, S1, BLK>;
    return split ? occupancy(k_igemm<MT, NT, KT, LA, LB, EpiRowMajor>)
                 : occupancy(k_igemm<MT, NT, KT, LA, LB, EpiNCHW>);
  }
  template <int MT, int NT, int KT>
  bool run() {
    const uint32_t OCp = pad4(g.OC), KK = g.k * g.k, kdim = KK * OCp;
    const uint32_t HW = g.H * g.W, N = g.B * HW;
    using LA = LdDenseRK<MT, KT>;
    using LB = LdPixRK<NT, KT, false, S1, BLK>;
    const typename LA::Params pa{wt, kdim, g.C, kdim, g.C * kdim};
    const typename LB::Params pb{gn, g.OH, g.OW, OCp, g.k, g.s, g.p, g.W, HW, N, kdim,
                                 g.B * g.OH * g.OW * OCp, make_fastdiv(HW), make_fastdiv(g.W),
                                 make_fastdiv(BLK ? KK : OCp), make_fastdiv(g.k)};
    const uint32_t kt = cdiv(kdim, KT);
    const EpiNCHW::Params pe{dx, nullptr, g.C, HW, N, 0, make_fastdiv(HW)};
    if (splits > 1) {
      const EpiRowMajor::Params pr{part, g.C, N, N, g.C * N};
      return launch<MT, NT, KT, LA, LB, EpiRowMajor>(pa, pb, pr, g.C, N, kt, splits,
                                                    "conv_backward_input") &&
             split_nchw(part, nullptr, dx, g.C, N, HW, splits, 0);
    }
    return launch<MT, NT, KT, LA, LB, EpiNCHW>(pa, pb, pe, g.C, N, kt, 1, "conv_backward_input");
  }
};

// One sub-pixel phase of a strided dX (s > 1).  The input pixels (b, ph +
// s*a, pw + s*c) receive only the taps kh = rh + s*jh (jh < nh), kw = rw +
// s*jw (jw < nw) with rh = (ph + p) mod s, whose output pixels are (a + qh -
// jh, c + qw - jw), qh = (ph + p - rh) / s: a stride-1 gather over the
// phase's own GH x GW grid with an nh x nw kernel.
struct PhaseGeom {
  uint32_t ph, pw, rh, rw, nh, nw, qh, qw, GH, GW;
};

template <bool BLK>
struct DxPhaseRun {
  const float* wt;
  const float* gn;
  float* dx;
  ConvGeom g;
  PhaseGeom q;
  template <int MT, int NT, int KT>
  int occ(bool) const {
    return occupancy(
        k_igemm<MT, NT, KT, LdDenseRK<MT, KT>, LdPixRK<NT, KT, false, true, BLK>, EpiNCHWPhase>);
  }
  template <int MT, int NT, int KT>
  bool run() {
    const uint32_t OCp = pad4(g.OC), KK = q.nh * q.nw, kdim = KK * OCp;
    const uint32_t GHW = q.GH * q.GW, N = g.B * GHW;
    using LA = LdDenseRK<MT, KT>;
    using LB = LdPixRK<NT, KT, false, true, BLK>;
    const typename LA::Params pa{wt, kdim, g.C, kdim, g.C * kdim};
    const typename LB::Params pb{gn, g.OH, g.OW, OCp, q.nw, 1, q.qh, q.GW, GHW, N, kdim,
                                 g.B * g.OH * g.OW * OCp, make_fastdiv(GHW), make_fastdiv(q.GW),
                                 make_fastdiv(BLK ? KK : OCp), make_fastdiv(q.nw),
                                 int(q.qw) - int(q.qh)};
    const EpiNCHWPhase::Params pe{dx, g.C, g.H, g.W, q.GW, GHW, N, g.s, q.ph, q.pw,
                                  make_fastdiv(GHW), make_fastdiv(q.GW)};
    return launch<MT, NT, KT, LA, LB, EpiNCHWPhase>(pa, pb, pe, g.C, N, cdiv(kdim, KT), 1,
                                                    "conv_backward_input");
  }
};

// dX of a strided convolution as its s*s sub-pixel phases: every input pixel
// multiplies only the taps that reach it, where the strided gather walks all
// k*k taps for every pixel and finds all but about 1/s^2 of them out of
// step.  Each phase gets its own filter re-layout (into wt, C * k*k * OCp
// floats) and GEMM, unsplit; phases that no tap reaches (k < s) are zero.
static bool phase_dx(const float* w, float* wt, const float* gn, float* dx, const ConvGeom& g) {
  const uint32_t s = g.s, OCp = pad4(g.OC);
  const bool blk = blocked_k(OCp);
  auto geom = [&](uint32_t ph, uint32_t pw) {
    PhaseGeom q{};
    q.ph = ph;
    q.pw = pw;
    q.GH = ph < g.H ? cdiv(g.H - ph, s) : 0;
    q.GW = pw < g.W ? cdiv(g.W - pw, s) : 0;
    q.rh = (ph + g.p) % s;
    q.rw = (pw + g.p) % s;
    q.nh = q.rh < g.k ? cdiv(g.k - q.rh, s) : 0;
    q.nw = q.rw < g.k ? cdiv(g.k - q.rw, s) : 0;
    q.qh = (ph + g.p - q.rh) / s;
    q.qw = (pw + g.p - q.rw) / s;
    return q;
  };
  bool empty = false;
  for (uint32_t ph = 0; ph < s; ++ph)
    for (uint32_t pw = 0; pw < s; ++pw) {
      const PhaseGeom q = geom(ph, pw);
      empty |= q.GH * q.GW > 0 && q.nh * q.nw == 0;
    }
  if (empty && !fill_zero(dx, size_t(g.B) * g.C * g.H * g.W)) return false;
  for (uint32_t ph = 0; ph < s; ++ph)
    for (uint32_t pw = 0; pw < s; ++pw) {
      const PhaseGeom q = geom(ph, pw);
      if (q.GH * q.GW == 0 || q.nh * q.nw == 0) continue;
      const uint32_t KK = q.nh * q.nw, kdim = KK * OCp, N = g.B * q.GH * q.GW;
      if (!permute_w(WPerm{w, wt, g.OC, g.C, KK, OCp, kdim, 1, blk ? 1 : 0, q.nw, g.k, s, q.rh,
                           q.rw}))
        return false;
      TileCfg c = choose(
          "DCE_TUNE_DX", g.C, N, kdim, 1, true,
          [&](const TileCfg& t) {
            return blk ? tiles_occ16(t, DxPhaseRun<true>{}) : tiles_occ16(t, DxPhaseRun<false>{});
          },
          true);
      narrow_short_k(c, "DCE_TUNE_DX", g.C, N, kdim);
      c.splits = 1;
      const bool ok = blk ? tiles_dispatch16(c, DxPhaseRun<true>{wt, gn, dx, g, q})
                          : tiles_dispatch16(c, DxPhaseRun<false>{wt, gn, dx, g, q});
      if (!ok) return false;
    }
  return true;
}

// Pointwise dX: dx[c][n] = sum_oc w[oc][c] dy[oc][n] (NCHW dy and dx; the
// filters re-laid [c][pad4(OC)]).
// WK: the A operand is the filters themselves, [OC][C] read as [k = oc][row
// = c] (C % 4 == 0); otherwise their re-layout [C][pad4(OC)].
template <bool WK>
struct DxPwRun {
  const float* wt;
  const float* dy;
  float* dx;
  float* part;
  ConvGeom g;
  uint32_t splits;
  template <int MT, int KT>
  using LAt = typename std::conditional<WK, LdDenseKR<MT, KT>, LdDenseRK<MT, KT>>::type;
  template <int MT, int NT, int KT>
  int occ(bool split) const {
    using LA = LAt<MT, KT>;
    using LB = LdNchwKR<NT, KT>;
    return split ? occupancy(k_igemm<MT, NT, KT, LA, LB, EpiRowMajor>)
                 : occupancy(k_igemm<MT, NT, KT, LA, LB, EpiNCHW>);
  }
  template <int MT, int NT, int KT>
  bool run() {
    const uint32_t OCp = pad4(g.OC), HW = g.H * g.W, N = g.B * HW;
    using LA = LAt<MT, KT>;
    using LB = LdNchwKR<NT, KT>;
    const typename LA::Params pa = WK ? typename LA::Params{wt, g.C, g.C, g.OC, g.OC * g.C}
                                      : typename LA::Params{wt, OCp, g.C, OCp, g.C * OCp};
    const NchwKRParams pb{dy, g.OC, HW, N, g.B * g.OC * HW, make_fastdiv(HW)};
    const uint32_t kt = cdiv(OCp, KT);
    const EpiNCHW::Params pe{dx, nullptr, g.C, HW, N, 0, make_fastdiv(HW)};
    if (splits > 1) {
      const EpiRowMajor::Params pr{part, g.C, N, N, g.C * N};
      return launch<MT, NT, KT, LA, LB, EpiRowMajor>(pa, pb, pr, g.C, N, kt, splits,
                                                    "conv_backward_input") &&
             split_nchw(part, nullptr, dx, g.C, N, HW, splits, 0);
    }
    return launch<MT, NT, KT, LA, LB, EpiNCHW>(pa, pb, pe, g.C, N, kt, 1, "conv_backward_input");
  }
};

// Pointwise dW: dw[oc][c] = sum_n dy[oc][n] x[c][n]; with db, x gets a row of
// ones (column C of the product is the bias gradient, written by the finish).
struct DwPwRun {
  const float* dy;
  const float* x;
  float* part;
  ConvGeom g;
  uint32_t N, splits;  // N = C, or C + 1 with the ones row
  bool trans;          // input channels as the product's rows (partials [z][c][oc])
  template <int MT, int NT, int KT>
  int occ(bool) const {
    return occupancy(k_igemm<MT, NT, KT, LdNchwRK<MT, KT>, LdNchwRK<NT, KT>, EpiRowMajor>);
  }
  template <int MT, int NT, int KT>
  bool run() {
    const uint32_t HW = g.H * g.W, K = g.B * HW;
    const NchwRKParams pa{dy, ones4(), g.OC, HW, K, g.B * g.OC * HW, 0xFFFFFFFFu, make_fastdiv(HW)};
    const NchwRKParams pb{x, ones4(), g.C, HW, K, g.B * g.C * HW, N > g.C ? g.C : 0xFFFFFFFFu,
                          make_fastdiv(HW)};
    const uint32_t zs = 4 * cdiv(size_t(g.OC) * N, 4);
    if (trans) {
      const EpiRowMajor::Params pe{part, N, g.OC, g.OC, zs};
      return launch<MT, NT, KT, LdNchwRK<MT, KT>, LdNchwRK<NT, KT>, EpiRowMajor>(
          pb, pa, pe, N, g.OC, cdiv(K, KT), splits, "conv_backward_filter");
    }
    const EpiRowMajor::Params pe{part, g.OC, N, N, zs};
    return launch<MT, NT, KT, LdNchwRK<MT, KT>, LdNchwRK<NT, KT>, EpiRowMajor>(
        pa, pb, pe, g.OC, N, cdiv(K, KT), splits, "conv_backward_filter");
  }
};

static bool conv_backward_pw(const float* dy, const float* x, const float* w, float* dw,
                             float* db, float* dx, const ConvGeom& g) {
  const uint32_t OCp = pad4(g.OC), HW = g.H * g.W, N = g.B * HW;
  const double fl = 2.0 * g.OC * g.C * double(N);
  ProfScope profAll("conv_bwd", fl * ((dw ? 1 : 0) + (dx ? 1 : 0)), 0.0);
  const uint32_t Ndw = g.C + (db ? 1u : 0u);
  TileCfg dwc{128, 128, 16, 1}, dxc{128, 128, 16, 1};
  size_t nP = 0, nW = 0, nQ = 0;
  // dW orientation with the fuller tile grid: expand layers (many more
  // output than input channels) put the few input channels on the narrow
  // rows.
  const bool dwT = tile_fill(Ndw, g.OC) > tile_fill(g.OC, Ndw) * 1.25;
  if (dw) {
    const uint32_t dM = dwT ? Ndw : g.OC, dN = dwT ? g.OC : Ndw;
    const uint32_t ntiles = cdiv(dM, pick_tile_m(dM)) * cdiv(dN, pick_tile(dN));
    dwc = choose(
        "DCE_TUNE_DW", dM, dN, N, ntiles <= 4 ? 1024 : 256, false,
        [&](const TileCfg& t) { return tiles_occ(t, DwPwRun{}); }, false, true);
    nP = al64(size_t(dwc.splits) * 4 * cdiv(size_t(g.OC) * Ndw, 4));
  }
  const bool wk = g.C % 4 == 0 && aligned16(w);  // dX reads the filters in place
  if (dx) {
    dxc = choose(
        "DCE_TUNE_DX", g.C, N, OCp, 8, true,
        [&](const TileCfg& t) {
          return wk ? tiles_occ16(t, DxPwRun<true>{}) : tiles_occ16(t, DxPwRun<false>{});
        },
        true);
    narrow_pw(dxc, "DCE_TUNE_DX", g.C, OCp);
    nW = wk ? 0 : al64(size_t(g.C) * OCp);
    nQ = dxc.splits > 1 ? size_t(dxc.splits) * g.C * N : 0;
  }
  float* ws = (nP + nW + nQ) ? workspace(nP + nW + nQ) : nullptr;
  if ((nP + nW + nQ) && !ws) return false;
  float* part = ws;
  float* wt = ws ? ws + nP : nullptr;
  float* qpart = wt ? wt + nW : nullptr;
  if (dw) {
    ProfScope prof("conv_dw", fl, 4.0 * (double(N) * g.OC + double(N) * g.C));
    if (!tiles_dispatch(dwc, DwPwRun{dy, x, part, g, Ndw, dwc.splits, dwT}) ||
        !dw_final(part, dw, g.OC, g.C, 1, Ndw, dwc.splits, dwT, BwdSide{}, db))
      return false;
  }
  if (dx) {
    if (!wk && !permute_w(WPerm{w, wt, g.OC, g.C, 1, OCp, OCp, 1, 0})) return false;
    ProfScope prof("conv_dx", fl, 4.0 * (double(N) * g.OC + double(N) * g.C));
    const bool ok = wk ? tiles_dispatch16(dxc, DxPwRun<true>{w, dy, dx, qpart, g, dxc.splits})
                       : tiles_dispatch16(dxc, DxPwRun<false>{wt, dy, dx, qpart, g, dxc.splits});
    if (!ok) return false;
  }
  return true;
}

uint32_t conv_g_layout(const ConvGeom& g) { return ps_x(g) ? kGLayoutPad : kGLayoutNhwc; }
bool conv_g_nhwc_pass(const ConvGeom& g) { return !ps_x(g) && !pw_x(g); }
uint32_t conv_g_pad_width(const ConvGeom& g) { return ps_geom(g).OWp; }

bool conv_backward(const float* dy, const float* y, const float* x, const float* x_nhwc,
                   const float* w, float* dw, float* db, float* dx, const ConvGeom& g,
                   const PreG* pre) {
  // Pointwise layers with no ReLU mask (and dW requested whenever db is: the
  // bias gradient is the dW product's ones column) read NCHW in place.
  if (pw_x(g)) {
    if (!y && (dw || !db)) {
      if (!operand_fits(size_t(g.B) * g.C * g.H * g.W, "conv_backward") ||
          !operand_fits(size_t(g.B) * g.OC * g.H * g.W, "conv_backward"))
        return false;
      return conv_backward_pw(dy, x, w, dw, db, dx, g);
    }
    x_nhwc = nullptr;  // the forward kept no copy: the general path builds its own
  }
  const uint32_t Cp = pad4(g.C), OCp = pad4(g.OC), KK = g.k * g.k;
  const uint32_t OHW = g.OH * g.OW, npix = g.B * OHW, HW = g.H * g.W;
  if (!operand_fits(size_t(npix) * OCp, "conv_backward") ||
      !operand_fits(xbuild_floats(g), "conv_backward") ||
      !operand_fits(size_t(g.C) * KK * OCp, "conv_backward"))
    return false;
  // Workspace carve-up: G (NHWC) and / or G_pad, db partials, the copy of x
  // if not kept by the forward, dW split-K partials, dX filters, dX split-K
  // partials.  Fewer than four input channels: x is stride-phase split (or,
  // for strides above 4, channel-packed) and the dW tap axis runs over KK * C
  // unpadded taps (Cx = C), otherwise over KK * pad4(C).
  const bool pk = packed_x(g), ps = ps_x(g);
  const uint32_t Cx = (pk || ps) ? g.C : Cp;
  const uint32_t npb = cdiv(OHW, 64);
  // The whole call as one family: the masked transpose of dy, the bias-grad
  // sum, any rebuilt copy of x, the filter re-layout and the split-K finishes
  // count with the GEMMs' FLOPs.
  const double callFlops = 2.0 * g.OC * g.C * KK * double(npix) * ((dw ? 1 : 0) + (dx ? 1 : 0));
  ProfScope profAll("conv_bwd", callFlops, 0.0);
  // The stride-phase dW reads the masked gradient on the padded pixel grid
  // (G_pad, which also yields the bias-gradient partials); dX reads the NHWC
  // G of the transpose pass.  Other layouts use the NHWC G for both.
  const PsGeom q = ps ? ps_geom(g) : PsGeom{};
  const bool useGpad = ps && (dw || (db && !dx)), useGnhwc = !ps || dx;
  // A G_pad made by dy's producer (with its bias-gradient partials) replaces
  // the masking pass that makes it.
  const bool preG = pre && pre->layout == kGLayoutPad && useGpad;
  // An NHWC G made by dy's producer (the batch-norm backward; no ReLU mask)
  // replaces the transpose pass.
  const bool preGn = pre && pre->layout == kGLayoutNhwc && !ps && !y;
  const uint32_t nchunk = ps ? cdiv(q.OHWp, kMaskChunk) : 0;
  const uint32_t dbRows = useGpad ? g.B * nchunk : g.B * npb;
  const uint32_t dwK = ps ? g.B * q.OHWp : npix;  // dW GEMM K extent (pixels)
  const size_t nG = (useGnhwc && !preGn) ? al64(size_t(npix) * OCp) : 0;
  const size_t nGp = (useGpad && !preG) ? al64(size_t(g.B) * g.OC * q.OHWp) : 0;
  const size_t nDb = (db && !preG && !preGn) ? al64(size_t(dbRows) * g.OC) : 0;
  const size_t nX = (dw && !x_nhwc) ? al64(xbuild_floats(g)) : 0;
  if (ps && !operand_fits(nGp, "conv_backward")) return false;
  TileCfg dwc{128, 128, 16, 1}, dxc{128, 128, 16, 1};
  size_t nP = 0, nW = 0, nQ = 0;
  bool dwT = false;
  if (dw) {
    // Orientation with the fuller tile grid; a grid of a few tiles gets more
    // split-K slices so that the whole chip works on it.
    const uint32_t taps = KK * Cx;
    dwT = tile_fill(taps, g.OC) > tile_fill(g.OC, taps) * 1.25;
    const uint32_t dM = dwT ? taps : g.OC, dN = dwT ? g.OC : taps;
    const uint32_t ntiles = cdiv(dM, pick_tile_m(dM)) * cdiv(dN, pick_tile(dN));
    dwc = choose(
        "DCE_TUNE_DW", dM, dN, dwK, ntiles <= 4 ? 1024 : 256, false,
        [&](const TileCfg& t) {
          DwRun r{};
          r.trans = dwT;
          r.pk = pk;
          r.ps = ps;
          return tiles_occ<true>(t, r);
        },
        false, true, !ps && !pk);
    nP = al64(size_t(dwc.splits) * 4 * cdiv(size_t(g.OC) * taps, 4));
  }
  // A dX at stride 3 or more runs as sub-pixel phases (phase_dx), each with
  // its own filter re-layout and no split: the strided gather would walk
  // s^2 times the taps that reach a pixel (AlexNet c1's dX at b128: 18.0 ->
  // 1.24 ms).  At stride 2 the gather's 4x is about what the phases' extra
  // launches and smaller, unsplit grids cost (ResNet-like layers of 0.4-7
  // GFLOP measured from 40 % faster to 65 % slower), so it stays.
  const bool phased = dx && g.s >= 3;
  if (dx && !phased) {
    const bool blk = blocked_k(OCp);
    dxc = choose(
        "DCE_TUNE_DX", g.C, g.B * HW, KK * OCp, 8, true,
        [&](const TileCfg& t) { return conv_variant_occ<DxRun>(g.s == 1, blk, t); }, true);
    narrow_short_k(dxc, "DCE_TUNE_DX", g.C, g.B * HW, KK * OCp);
    nQ = dxc.splits > 1 ? size_t(dxc.splits) * g.C * g.B * HW : 0;
  }
  if (dx) nW = al64(size_t(g.C) * KK * OCp);
  float* ws = workspace(nG + nGp + nDb + nX + nP + nW + nQ);
  if (!ws) return false;
  float* gn = ws;
  float* gp = gn + nG;
  float* dbPart = db ? gp + nGp : nullptr;
  float* xs = gp + nGp + nDb;
  float* part = xs + nX;
  float* wt = part + nP;
  float* qpart = wt + nW;
  if (preG) {
    gp = const_cast<float*>(pre->g);
    if (db) dbPart = const_cast<float*>(pre->db);
  }
  if (preGn) {
    gn = const_cast<float*>(pre->g);
    if (db) dbPart = const_cast<float*>(pre->db);
  }

  if (useGpad && !preG) {
    bool ok = false;
    mask_pad(dy, y, gp, dbPart, g, &ok);
    if (!ok) return false;
  }
  // The dX filter re-layout rides in the G pass launch (dX always has the
  // NHWC G), the bias-gradient sum in the dW finishing launch.
  const WPerm dxPerm{w, wt, g.OC, g.C, KK, OCp, KK * OCp, 1, dx && blocked_k(OCp) ? 1 : 0};
  uint32_t npbGot = npb;
  if (useGnhwc && !preGn &&
      !to_nhwc_masked(dy, y, gn, useGpad ? nullptr : dbPart, g.B, g.OC, OHW, &npbGot,
                      dx && !phased ? dxPerm : WPerm{}))
    return false;
  // With the producer's G the dX filter re-layout rides in the dW finish
  // (which runs before dX), or runs by itself when no dW is asked for.
  const bool permInFinish = preGn && dx && !phased && dw;
  if (preGn && dx && !phased && !dw && !permute_w(dxPerm)) return false;
  const uint32_t dbRowsGot =
      (preG || preGn) ? pre->dbRows : (useGpad ? dbRows : g.B * npbGot);
  if (db && !dw) {
    hipLaunchKernelGGL(k_rowsum, dim3(g.OC), dim3(256), 0, stream(), dbPart, db, dbRowsGot);
    if (!check_launch("bias_grad")) return false;
  }
  auto dx_chain = [&]() {
    ProfScope prof("conv_dx", 2.0 * g.OC * g.C * KK * double(npix),
                   4.0 * (double(npix) * OCp + double(g.B) * g.C * g.H * g.W));
    if (phased) return phase_dx(w, wt, gn, dx, g);
    return conv_variant<DxRun>(g.s == 1, dxPerm.blocked != 0, dxc, wt, gn, dx, qpart, g,
                               dxc.splits);
  };
  auto dw_gemm = [&]() {
    const float* xn = x_nhwc;
    if (!xn) {
      const bool built = ps ? to_ps(x, xs, g)
                            : (pk ? to_pk(x, xs, g) : to_nhwc(x, xs, g.B, g.C, g.H, g.W));
      if (!built) return false;
      xn = xs;
    }
    ProfScope prof("conv_dw", 2.0 * g.OC * g.C * KK * double(npix),
                   4.0 * (double(npix) * OCp + double(g.B) * g.H * g.W * Cp + double(g.OC) * KK * Cp));
    return tiles_dispatch<true>(dwc, DwRun{ps ? gp : gn, xn, part, g, dwc.splits, dwT, pk, ps});
  };
  auto dw_finish = [&]() {
    BwdSide side{};
    if (db) {
      side.dbPart = dbPart;
      side.db = db;
      side.dbRows = dbRowsGot;
      side.nRow = g.OC;
    }
    // The stride-phase taps are already in the filters' (c, kh, kw) order:
    // the finish is a plain split sum (one channel of C*KK taps).
    return ps ? dw_final(part, dw, g.OC, 1, KK * g.C, 1, dwc.splits, dwT, side)
              : dw_final(part, dw, g.OC, g.C, KK, Cx, dwc.splits, dwT, side, nullptr,
                         permInFinish ? dxPerm : WPerm{});
  };
  if (dw && !(dw_gemm() && dw_finish())) return false;
  if (dx && !dx_chain()) return false;
  return true;
}

}  // namespace dce
