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
  uint32_t tag;
  uint32_t meta[5];
};
constexpr uint32_t kPoolTag = 0x9001u;
constexpr uint32_t kNhwcTag = 0x9002u;

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

// Handle validation: returns the Buffer or nullptr (error set) for NULL,
// released or foreign handles.
Buffer* as_buffer(void* h, const char* what);
void* create_buffer(const float* host, uint32_t count);
void release_buffer(void* h);

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
  __device__ __forceinline__ float ld1(uint32_t off) const {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off * 4u, 0, 0));
  }
};

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
// y = act(conv(x, w) + bias) in NCHW.  x_nhwc_keep, when not null, receives
// the NHWC copy of x (nhwc_floats(B, C, H, W)) for a later backward.
bool conv_forward(const float* x, float* x_nhwc_keep, const float* w, const float* bias,
                  float* y, const ConvGeom& g, uint32_t act);
// dW[OC, C, k, k], db[OC], dX (NCHW) from G = dy masked by y (> 0 kept; y may
// be null: no mask).  Any of dw, db, dx may be null (not requested).
// x_nhwc, when not null, is the NHWC copy produced by conv_forward.
bool conv_backward(const float* dy, const float* y, const float* x, const float* x_nhwc,
                   const float* w, float* dw, float* db, float* dx, const ConvGeom& g);
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

}  // namespace dce
