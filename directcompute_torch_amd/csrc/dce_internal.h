// Internal interfaces shared by the libdcengine translation units.
// Nothing here is part of the C ABI (that is include/dcengine.h).
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstddef>

namespace dce {

// ---------------------------------------------------------------------------
// Buffer record behind every opaque handle of the C ABI.
// ---------------------------------------------------------------------------
constexpr uint32_t kMagicLive = 0xDCB0F1A7u;
constexpr uint32_t kMagicPooled = 0xDCB0900Du;
constexpr uint32_t kMagicDead = 0xDEADB0F5u;

struct Buffer {
  float* ptr;         // device pointer (256-byte aligned, hipMalloc)
  uint32_t count;     // element count in floats (the reference's u32 size)
  int refCount;
  uint32_t magic;
  // Producer metadata, reset whenever the buffer is handed out again:
  //  kPoolTag: indices of MaxPoolForwardFused, meta = {H, W, k, s}, so the
  //            backward can run as a deterministic gather;
  //  kNhwcTag: channel-innermost copy of a conv input kept by
  //            ConvForwardFused as its "im2col" handle, meta = {B, C, H, W, Cp}.
  //  kReluOutTag: output of a ReLU ConvForwardFused whose backward reads its
  //            masked gradient on the padded pixel grid (fewer than 4 input
  //            channels), meta = {kGLayoutPad, B, OC, OH, OW};
  //  kPoolOutTag: output of MaxPoolForwardFused (its values are the
  //            windows' maxima, which the masked max-pool backward reads);
  //  kGradGTag: gradient written by MaxPoolBackwardFused for a ReLU conv
  //            output (src): `side` holds that conv's masked gradient G in
  //            the layout its backward reads, followed by bias-gradient
  //            partials, meta = {layout, B, OC, OH, OW}, aux32 = partial rows;
  //  kBnStatsTag: output of a ConvForwardFused with no activation whose GEMM
  //            left the batch-norm statistics of its values: `side` holds
  //            the per-channel double sums of y and y*y as [C][pieces][2],
  //            meta = {B, C, H*W, H, W}, aux32 = pieces; meta[3..4] are 0
  //            unless the conv's backward reads its gradient as an NHWC G
  //            (then batchnorm_backward_dx over y makes that G);
  //  kGradGTag also marks the dx of batchnorm_backward_dx over such a y:
  //            side = [NHWC G | bias-gradient partials], src = null;
  //  kBnOutTag: output z of batchnorm_forward; key = that call's gamma
  //            buffer (a key only: the layer), meta = {N, C, S}, aux32b =
  //            the bits of eps; src = x (when it carries kBnStatsTag) and
  //            aux = the batch mean (kBnMomentTag) it normalised with; when
  //            the forward also stored act(z) for the activation that
  //            followed this layer last time, side = that buffer, aux32 = 1
  //            (relu) or 2 (relu6);
  //  kBnMomentTag: batch mean and variance of batchnorm_mean_var; the
  //            mean's src = the variance;
  //  kBnGradPartTag: dz of relu_grad / relu6_grad over such a z: side holds
  //            the partial sums of batchnorm_backward_reduce over (x, dz)
  //            ([C][pieces][2] doubles), src = x, aux = mean, meta = {N, C,
  //            S}, aux32 = pieces, aux32b = the bits of eps.
  // A tag is dropped (drop_tag) whenever the buffer is written by anything
  // but its producer, and when the buffer goes back to the pool.
  uint32_t tag;
  uint32_t meta[5];
  // Tag identity: a fresh value of a global counter each time a tag is set,
  // so that a link to another buffer (src, aux) stays valid only while that
  // buffer still carries the tag it had when the link was made (records are
  // recycled, never deleted).
  uint64_t gen;
  Buffer* src;      // kPoolTag: the pooled input (ReLU conv output); kGradGTag: that conv output
  uint64_t srcGen;
  Buffer* aux;      // kPoolTag: the pooled output
  uint64_t auxGen;
  Buffer* side;     // kGradGTag: owned buffer [G | bias-gradient partials]; kBnStatsTag: the sums
  uint32_t aux32;
  uint32_t aux32b;
  const void* key;  // kBnOutTag: the layer's gamma buffer
};
constexpr uint32_t kPoolTag = 0x9001u;
constexpr uint32_t kNhwcTag = 0x9002u;
constexpr uint32_t kReluOutTag = 0x9003u;
constexpr uint32_t kPoolOutTag = 0x9004u;
constexpr uint32_t kGradGTag = 0x9005u;
constexpr uint32_t kBnStatsTag = 0x9006u;
constexpr uint32_t kBnOutTag = 0x9007u;
constexpr uint32_t kBnMomentTag = 0x9008u;
constexpr uint32_t kBnGradPartTag = 0x9009u;
// Layouts of a conv backward's masked gradient G.
constexpr uint32_t kGLayoutPad = 1;   // [B*OC][OH][pad4(OW)], zero past OW (stride-phase dW)
constexpr uint32_t kGLayoutNhwc = 2;  // [B*OH*OW][pad4(OC)] (the transpose pass)

// Floats of G in `layout` for a conv output [B][C][H][W], rounded up to 64
// (the bias-gradient partials follow it in a kGradGTag side buffer).
inline size_t g_side_floats(uint32_t layout, uint32_t B, uint32_t C, uint32_t H, uint32_t W) {
  const size_t n = layout == kGLayoutNhwc ? size_t(B) * H * W * ((C + 3u) & ~3u)
                                          : size_t(B) * C * H * ((W + 3u) & ~3u);
  return (n + 63) & ~size_t(63);
}

// batchnorm_backward_dx of one element (nn_batchnorm_backward_dx.hlsl:26-38),
// shared by every kernel that computes it so that they agree bit for bit:
// rstd = 1 / sqrt(var + eps), m = N * S.
__device__ __forceinline__ float bn_dx_elem(float x, float dy, float mu, float rstd, float g,
                                            float dg, float db, float m) {
  const float xh = (x - mu) * rstd;
  return (g * rstd) * (dy - (db + xh * dg) / m);
}

// Does buffer `b` still carry tag `tag` of generation `gen`?
inline bool tag_alive(const Buffer* b, uint32_t tag, uint64_t gen) {
  return b && b->magic == kMagicLive && b->tag == tag && b->gen == gen;
}

// A bounds-carrying view used by the RunShader-compatible kernels: reads past
// `n` return 0 and writes past `n` are dropped, like D3D11 structured buffers.
struct Buf {
  float* p;
  uint32_t n;
};

// Engine state accessors (dce_engine.hip).
hipStream_t stream();
int num_cus();
bool ensure_init();
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
bool check_launch(const char* what);

// Persistent scratch space in device memory, reused by consecutive launches on
// the single in-order stream.  Grows on demand (the old block is freed only
// after the stream drains).  Returns nullptr (error set) on failure.
float* workspace(size_t floats);
// Four floats of 1.0 in device memory (set at InitEngine), for loaders that
// feed a row of ones to a GEMM.
const float* ones4();

// Handle validation: returns the Buffer or nullptr (error set) for NULL,
// released or foreign handles.
Buffer* as_buffer(void* h, const char* what);
void* create_buffer(const float* host, uint32_t count);
void release_buffer(void* h);
// Tag buffer y (B x C x S floats) kBnStatsTag: `side` (owned by y from now
// on) holds the per-channel double sums of y and y*y, [C][pieces][2].  H, W:
// the plane of a conv output whose backward reads an NHWC G (else 0, 0).
void tag_bn_stats(void* y, void* side, uint32_t B, uint32_t C, uint32_t S, uint32_t pieces,
                  uint32_t H = 0, uint32_t W = 0);
// The activation (1 relu, 2 relu6, 0 none seen) that last followed the batch
// norm whose gamma buffer is `gamma`.
uint32_t bn_act_guess(const void* gamma);
// Tag z (a batchnorm_forward output over x with batch statistics mean /
// var) kBnOutTag; side (may be null) holds act(z), owned by z from now on.
void tag_bn_out(void* z, void* x, void* mean, void* gamma, void* side, uint32_t act,
                uint32_t N, uint32_t C, uint32_t S, float eps);
// Tag the batch statistics of batchnorm_mean_var kBnMomentTag.
void tag_bn_moments(void* mean, void* var);
// For relu_grad / relu6_grad over z: when z is a batchnorm_forward output
// whose x and statistics are unchanged since, the device pointers of x, mean
// and var, the shape and eps, and true.
struct BnLink {
  const float* x;
  const float* mean;
  const float* var;
  uint32_t N, C, S;
  float eps;
};
bool bn_link_of(void* z, BnLink* out);
// Tag dz kBnGradPartTag with the partial sums in `side` (owned by dz from
// now on), made over z's batch norm (bn_link_of).
void tag_bn_grad_part(void* dz, void* z, void* side, uint32_t pieces);
// batchnorm_backward_reduce(x, dy, mean, var, eps) over N, C, S: the partial
// sums dy carries for exactly these operands, or null.
const double* bn_grad_part_of(void* dy, void* x, void* mean, void* var, uint32_t N, uint32_t C,
                              uint32_t S, float eps, uint32_t* pieces);
// relu (act 1) / relu6 (act 2) of n elements from z into a: when z carries
// that activation already stored for all n elements of a, a takes that
// storage over (a's own goes back to the pool) and true is returned; the
// activation is remembered for z's layer either way.
bool bn_act_adopt(void* z, void* a, uint32_t act, uint32_t n);
// Tag dx kGradGTag with an NHWC G side buffer (owned by dx from now on) for
// the conv whose output has B x C channels of H x W; rows = db partial rows.
void tag_grad_g_nhwc(void* dx, void* side, uint32_t B, uint32_t C, uint32_t H, uint32_t W,
                     uint32_t rows);

// ---------------------------------------------------------------------------
// Fast unsigned division by a run-time constant (numerators < 2^31).
// q = (umulhi(n, mul) + n) >> shr, with mul/shr computed on the host.
// ---------------------------------------------------------------------------
struct FastDiv {
  uint32_t d, mul, shr;
};
FastDiv make_fastdiv(uint32_t d);

__device__ __forceinline__ uint32_t fdiv(uint32_t n, FastDiv f) {
  return (__umulhi(n, f.mul) + n) >> f.shr;
}

// ---------------------------------------------------------------------------
// Operand view through a buffer resource.  The descriptor's range check makes
// a load at or past num_records return zeros, so a padding or out-of-image
// element is read by moving its offset to kOob instead of branching around
// the load: a thread's loads are issued back to back, with no exec-mask
// juggling between them.  Offsets are in floats; callers admit operands of
// fewer than kOob floats (2 GiB), so kOob (+ any tile offset) is always past
// num_records.
// ---------------------------------------------------------------------------
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
constexpr uint32_t kOob = 0x20000000u;
struct BRes {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ void init(const float* p, uint32_t nfloats) {
    // Word 3 = 0x00020000: 32-bit data format, no swizzle, raw (stride 0).
    r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), 0, int(nfloats * 4u), 0x00020000);
  }
  // The builtins return raw 32-bit words; the bit casts keep them bits.
  __device__ __forceinline__ f4 ld4(uint32_t off) const {
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, off * 4u, 0, 0));
  }
  // Nontemporal form (the NT cache-policy bit), for passes larger than the MALL.
  __device__ __forceinline__ f4 ld4nt(uint32_t off) const {
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, off * 4u, 0, 2));
  }
  __device__ __forceinline__ float ld1(uint32_t off) const {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off * 4u, 0, 0));
  }
  __device__ __forceinline__ f2 ld2(uint32_t off) const {
    return __builtin_bit_cast(f2, __builtin_amdgcn_raw_buffer_load_b64(r, off * 4u, 0, 0));
  }
  __device__ __forceinline__ f2 ld2nt(uint32_t off) const {
    return __builtin_bit_cast(f2, __builtin_amdgcn_raw_buffer_load_b64(r, off * 4u, 0, 2));
  }
  // 16 bytes per lane straight into LDS: the wave's lanes fill 64 consecutive
  // 16-byte slots from `lds` (wave-uniform) in lane order; an offset past
  // num_records writes zeros.  Completion is tracked by vmcnt.
  __device__ __forceinline__ void ld4_lds(uint32_t off, float* lds) const {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)lds, 16, off * 4u, 0, 0, 0);
  }
};

// ---------------------------------------------------------------------------
// 8- and 16-byte accesses at 4-byte alignment (rows of odd length).  The GPU
// runs with unaligned memory access enabled, so these stay single
// global_load/store_dwordx2/x4 instructions; memcpy states the alignment
// without the undefined behaviour of a misaligned vector-pointer cast.
// ---------------------------------------------------------------------------
template <class V>
__device__ __forceinline__ V ldu(const void* p) {
  V v;
  __builtin_memcpy(&v, p, sizeof(V));
  return v;
}
template <class V>
__device__ __forceinline__ void stu(void* p, const V& v) {
  __builtin_memcpy(p, &v, sizeof(V));
}

// ---------------------------------------------------------------------------
// Streaming accesses: 16-byte loads and stores with the nontemporal cache
// policy, for passes over more data than the 256 MB MALL (Infinity Cache)
// holds.  On MI355X they sustain more HBM bandwidth than the default policy
// (read streams 89% against 79% of 8 TB/s, a read-read-write update 77%
// against 69%, measured on 1.2 GB buffers).  Below that size the default
// policy wins: the producer's output is still in the MALL when the next
// kernel reads it.
// ---------------------------------------------------------------------------
// The threshold is a run-time value (default kStreamBytes) so that both
// template instances of every streaming kernel can be checked at small sizes
// (SetStreamingThreshold).
constexpr double kStreamBytes = 256.0 * 1024 * 1024;
extern double g_streamBytes;
inline bool stream_nt(double bytes) { return bytes > g_streamBytes; }
__device__ __forceinline__ f4 ldnt4(const float* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
}
__device__ __forceinline__ void stnt4(float* p, f4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<f4*>(p));
}
// The policy is a template parameter: a run-time choice between two loads of
// one address lets the compiler merge them and drop the nontemporal hint.
template <bool NT>
__device__ __forceinline__ f4 ld4s(const float* p) {
  if constexpr (NT)
    return ldnt4(p);
  else
    return *reinterpret_cast<const f4*>(p);
}
template <bool NT>
__device__ __forceinline__ void st4s(float* p, f4 v) {
  if constexpr (NT)
    stnt4(p, v);
  else
    *reinterpret_cast<f4*>(p) = v;
}

// ---------------------------------------------------------------------------
// Workgroup order.  The dispatcher hands consecutive workgroup ids to the 8
// XCDs in turn, and each XCD has its own L2.  xcd_block_id() renumbers a 1-D
// grid so that each XCD runs a contiguous range of logical ids: neighbouring
// logical blocks that share cache lines (rows of odd length, halos) then hit
// the same L2 instead of fetching the line once per XCD.
// ---------------------------------------------------------------------------
// The form with a count renumbers the first nwg workgroups of a grid whose
// remaining workgroups do other work.
__device__ __forceinline__ uint32_t xcd_block_id(uint32_t nwg) {
  const uint32_t L = blockIdx.x;
  const uint32_t q = nwg >> 3, r = nwg & 7, x = L & 7;
  return x * q + min(x, r) + (L >> 3);
}
__device__ __forceinline__ uint32_t xcd_block_id() { return xcd_block_id(gridDim.x); }

// Workgroups of `threads` threads of one kernel that a CU holds at once (from
// the runtime, cached per kernel address: kernels of one signature share the
// template instance).
int blocks_per_cu_raw(const void* kernel, int threads);
template <class Kern>
int blocks_per_cu(Kern kernel, int threads) {
  return blocks_per_cu_raw(reinterpret_cast<const void*>(kernel), threads);
}

// ---------------------------------------------------------------------------
// Wave-wide reductions over the 64 lanes of a wavefront, without LDS.  Inside
// each row of 16 lanes, DPP moves combine lanes: quad_perm [1,0,3,2] and
// [2,3,0,1] (every lane holds its quad's total), row_half_mirror (its 8-lane
// half-row's), row_mirror (its row's).  ds_swizzle with xor mask 16 then
// combines neighbouring rows inside each 32-lane half, and readlane 0 / 32
// joins the halves.  Every step pairs each lane with a partner holding the
// mirror-image partial, so all lanes carry bit-identical values throughout and
// the result (returned in every lane) does not depend on the lane.  All 64
// lanes must be active.
// ---------------------------------------------------------------------------
namespace xl {
constexpr int kQuadSwap1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kQuadSwap2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kHalfMirror = 0x141; // row_half_mirror
constexpr int kRowMirror = 0x140;  // row_mirror
constexpr int kSwzXor16 = 0x401F;  // ds_swizzle bit mode: and 0x1F, or 0, xor 0x10

template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ uint32_t swz32(uint32_t v) {
  return uint32_t(__builtin_amdgcn_ds_swizzle(int(v), kSwzXor16));
}
__device__ __forceinline__ uint32_t rdl32(uint32_t v, int lane) {
  return uint32_t(__builtin_amdgcn_readlane(int(v), lane));
}
// A value moved lane to lane as 32-bit words.
template <class T>
struct Words;
template <>
struct Words<float> {
  template <class F>
  __device__ static __forceinline__ float map(float v, F f) {
    return __builtin_bit_cast(float, f(__builtin_bit_cast(uint32_t, v)));
  }
};
template <>
struct Words<double> {
  template <class F>
  __device__ static __forceinline__ double map(double v, F f) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = f(uint32_t(u)), hi = f(uint32_t(u >> 32));
    return __builtin_bit_cast(double, (hi << 32) | lo);
  }
};
template <int CTRL, class T>
__device__ __forceinline__ T dpp(T v) {
  return Words<T>::map(v, [](uint32_t w) { return dpp32<CTRL>(w); });
}
template <class T>
__device__ __forceinline__ T swz(T v) {
  return Words<T>::map(v, [](uint32_t w) { return swz32(w); });
}
template <class T>
__device__ __forceinline__ T readlane(T v, int lane) {
  return Words<T>::map(v, [lane](uint32_t w) { return rdl32(w, lane); });
}
}  // namespace xl

struct OpAddR {
  template <class T>
  __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct OpMaxR {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

// Combine of the 8 lanes 8j..8j+7 (every lane of the group gets it).
template <class T, class Op = OpAddR>
__device__ __forceinline__ T group8_reduce(T v, Op op = Op()) {
  v = op(v, xl::dpp<xl::kQuadSwap1>(v));
  v = op(v, xl::dpp<xl::kQuadSwap2>(v));
  return op(v, xl::dpp<xl::kHalfMirror>(v));
}
template <class T, class Op = OpAddR>
__device__ __forceinline__ T wave_reduce(T v, Op op = Op()) {
  v = group8_reduce(v, op);
  v = op(v, xl::dpp<xl::kRowMirror>(v));
  v = op(v, xl::swz(v));
  return op(xl::readlane(v, 0), xl::readlane(v, 32));
}

// Block-wide sum (256 threads) in double, in a fixed order; result valid in
// thread 0.  sh: 4 doubles of shared memory.
__device__ __forceinline__ double block_sum256(double v, double* sh) {
  v = wave_reduce(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) sh[w] = v;
  __syncthreads();
  double s = 0;
  if (threadIdx.x == 0) s = (sh[0] + sh[1]) + (sh[2] + sh[3]);
  return s;
}

// ---------------------------------------------------------------------------
// Convolution geometry (NCHW, square kernels, zero padding, floor mode).
// ---------------------------------------------------------------------------
struct ConvGeom {
  uint32_t B, C, H, W, OC, k, s, p, OH, OW;
};

inline uint32_t pad4(uint32_t c) { return (c + 3u) & ~3u; }

// Implicit-GEMM MFMA launchers (dce_igemm.hip).  All pointers are device
// pointers with at least the extents implied by the geometry.
//
// Channel-innermost ("NHWC") copy of an NCHW activation with the channel
// count padded to pad4(C) (zeros): out[((b*H + h)*W + w)*Cp + c].
size_t nhwc_floats(uint32_t B, uint32_t C, uint32_t H, uint32_t W);
bool to_nhwc(const float* x, float* out, uint32_t B, uint32_t C, uint32_t H, uint32_t W);
// The copy of x that a convolution's GEMMs read: NHWC as above, or, for
// fewer than four input channels, channel-packed and zero-padded by the
// convolution's padding ([B][H + 2p][W + 2p][C], unpadded C).  xcopy_floats
// is its size and xcopy_tag a value that differs between the two layouts
// (and between paddings of the packed one).
bool packed_x(const ConvGeom& g);
size_t xcopy_floats(const ConvGeom& g);
uint32_t xcopy_tag(const ConvGeom& g);
// Batch-norm statistics of a conv forward's output, asked for by the caller:
// when the forward's GEMM can leave them (no activation, stride 1, no split,
// x of at least 4 channels or a pointwise layer) it calls get(ctx, pieces)
// for a buffer of OC * pieces * 2 doubles, writes the per-channel sums of y
// and y*y there ([oc][piece][2]) and sets `pieces`; otherwise pieces is 0.
struct ConvStatsReq {
  double* (*get)(void* ctx, uint32_t pieces);
  void* ctx;
  uint32_t pieces;
};
// y = act(conv(x, w) + bias) in NCHW.  x_nhwc_keep, when not null, receives
// the copy of x (xcopy_floats(g) floats) for a later backward.
bool conv_forward(const float* x, float* x_nhwc_keep, const float* w, const float* bias,
                  float* y, const ConvGeom& g, uint32_t act, ConvStatsReq* st = nullptr);
// The layout of G that conv_backward reads for this geometry (kGLayoutPad or
// kGLayoutNhwc), and the padded row width of kGLayoutPad.
uint32_t conv_g_layout(const ConvGeom& g);
// Does the backward of this conv without a ReLU mask make an NHWC G (the
// transpose pass)?  Not for pointwise or fewer-than-4-channel layers.
bool conv_g_nhwc_pass(const ConvGeom& g);
// batchnorm_backward_dx (x, dy, the statistics and gamma, dgamma, dbeta of C
// channels over B planes of HW) writing dx and, with it, the NHWC G of dx
// (dx transposed to [B*HW][pad4(C)]) and the bias-gradient partials that a
// conv backward's transpose pass would make: g_side_floats(kGLayoutNhwc, ...)
// floats of G, then C x rows partials.  rows = bn_dx_g_rows(B, C, HW).
uint32_t bn_dx_g_rows(uint32_t B, uint32_t C, uint32_t HW);
bool bn_dx_g(const float* x, const float* dy, const float* mean, const float* var,
             const float* gamma, const float* dg, const float* db, float eps, float* dx,
             float* g, float* dbPart, uint32_t B, uint32_t C, uint32_t HW);
uint32_t conv_g_pad_width(const ConvGeom& g);
// A masked gradient G made by the producer of dy (the max-pool backward):
// g in `layout` (kGLayoutPad), db = bias-gradient partials [OC][dbRows].
struct PreG {
  uint32_t layout;  // kGLayoutPad (a ReLU conv's masked G) or kGLayoutNhwc (no mask)
  const float* g;
  const float* db;
  uint32_t dbRows;
};
// dW[OC, C, k, k], db[OC], dX (NCHW) from G = dy masked by y (> 0 kept; y may
// be null: no mask).  Any of dw, db, dx may be null (not requested).
// x_nhwc, when not null, is the copy of x produced by conv_forward.  pre, when
// not null, is G (of dy masked by y) already made: the pass that would make
// it from dy and y is skipped.
bool conv_backward(const float* dy, const float* y, const float* x, const float* x_nhwc,
                   const float* w, float* dw, float* db, float* dx, const ConvGeom& g,
                   const PreG* pre = nullptr);
// C[M,N] = op(A)·op(B); flags bit0: A stored K×M, bit1: B stored N×K.
bool gemm(const float* a, const float* b, float* c, uint32_t M, uint32_t K,
          uint32_t N, uint32_t flags);

// Profiling hooks (dce_engine.hip): kernel-family timing with HIP events on
// the engine stream.  `family` is a short static string.
struct ProfScope {
  const char* family;
  double flops;
  double bytes;
  void* ev0;
  ProfScope(const char* fam, double fl, double by);
  ~ProfScope();
};

// Elementwise / reduction launchers used by the fused C entry points
// (dce_kernels.hip).
bool fill_zero(float* p, size_t n);
bool maxpool_forward(const float* x, float* out, float* idx, uint32_t B, uint32_t C,
                     uint32_t H, uint32_t W, uint32_t k, uint32_t s, uint32_t OH,
                     uint32_t OW);
bool maxpool_backward(const float* dz, const float* idx, float* dx, uint32_t B,
                      uint32_t C, uint32_t OH, uint32_t OW, uint32_t xcount,
                      uint32_t H, uint32_t W, uint32_t k, uint32_t s);
// Max-pool backward over a ReLU conv output (stride 2, windows of 2 or 3):
// dx as maxpool_backward, and the conv backward's masked gradient G of dx
// (masked where the window maximum `pooled` is <= 0, which is the conv
// output at the window's argmax) on the padded pixel grid (layout
// kGLayoutPad, rows of gw = pad4(W) floats), with bias-gradient partials
// db[C][rows]; maxpool_backward_g_rows gives rows.  maxpool_backward_g_ok
// tells whether a geometry and layout are supported.
bool maxpool_backward_g_ok(uint32_t C, uint32_t H, uint32_t W, uint32_t OH, uint32_t OW,
                           uint32_t k, uint32_t s, uint32_t layout);
uint32_t maxpool_backward_g_rows(uint32_t B, uint32_t H, uint32_t W, uint32_t layout);
bool maxpool_backward_g(const float* dz, const float* idx, const float* pooled, float* dx,
                        float* g, float* db, uint32_t B, uint32_t C, uint32_t OH, uint32_t OW,
                        uint32_t H, uint32_t W, uint32_t k, uint32_t layout, uint32_t gw);

// Shader registry (dce_kernels.hip).
struct Dispatch {
  void** srvs;
  uint32_t nS;
  void** uavs;
  uint32_t nU;
  const uint32_t* groups;
  const uint8_t* cb;
  uint32_t cbBytes;
};
typedef bool (*ShaderFn)(const Dispatch&);
struct ShaderEntry {
  const char* name;
  ShaderFn fn;
};
const ShaderEntry* find_shader(const char* name);
// The entry at address p, or nullptr when p is not an element of the registry.
const ShaderEntry* shader_entry(const void* p);

// Multi-tensor optimiser launchers (dce_optim.hip).
bool sgd_multi(void** params, void** grads, const uint32_t* sizes, uint32_t n,
               float lr, float clip);
bool grad_norm_multi(void** grads, const uint32_t* sizes, uint32_t n, float max_norm,
                     float* d_norm_scale /* device [2] */);
bool sgd_scaled_multi(void** params, void** grads, const uint32_t* sizes, uint32_t n,
                      float lr, const float* d_norm_scale);
bool scale_grads_multi(void** grads, const uint32_t* sizes, uint32_t n,
                       const float* d_norm_scale);
bool adam_multi(void** params, void** grads, void** m, void** v, const uint32_t* sizes,
                uint32_t n, float step, float b1, float b2, float eps, float wd, float clip);
// Adam with the step counter and step size in device memory state[0..1]
// (t_set > 0: set the counter to t_set and the step size to step_host; 0:
// advance the counter by one and evaluate the step size on the device).
bool adam_counted_multi(void** params, void** grads, void** m, void** v,
                        const uint32_t* sizes, uint32_t n, float* state, uint32_t t_set,
                        float step_host, double lr, double b1, double b2, float eps, float wd,
                        float clip);
// Static-scratch norm clip (no allocation): noalloc_setup records the scratch
// array's address on `device` (which must be current); clip_grad_norm_noalloc
// returns the norm, NaN while capturing, or -1 with the error set.
bool noalloc_setup(int device);
float clip_grad_norm_noalloc(int device, void** grads, const uint32_t* sizes, uint32_t n,
                             float max_norm, bool capturing);

}  // namespace dce
