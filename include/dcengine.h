/*
 * dcengine.h -- C ABI of libdcengine.so, the MI355X (gfx950) backend that
 * replaces engine.dll of raviadi12/directcompute_torch.
 *
 * Every entry point below has the name, argument order and meaning of the
 * engine.dll export cited beside it (engine.cpp:line), as bound by ctypes in
 * nn_engine.py:42-121, so the reference's host code can load this library in
 * place of engine.dll.  Differences in behaviour are listed per function.
 *
 * Conventions kept from the reference:
 *   - a buffer handle is an opaque void* to a record {device ptr, u32 element
 *     count (floats), refcount}; every size is a count of 32-bit floats;
 *   - all work is queued in order on ONE device stream (the D3D11 immediate
 *     context analogue); only ReadBuffer, SyncGPU and SGDBatchClipped block;
 *   - failures never abort the process: functions return false / NULL /
 *     do nothing, and (addition) the reason is kept for GetLastErrorString();
 *   - single host thread: like engine.dll, the library is not re-entrant.
 */
#ifndef DCENGINE_H
#define DCENGINE_H

#include <stdint.h>
#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- device -- */

/* engine.cpp:61 InitEngine.  Selects HIP device 0 (or $DCE_DEVICE), creates
 * the engine stream.  Idempotent; false when no HIP device is usable. */
bool InitEngine(void);

/* engine.cpp:132 GetGPUInfo.  160-byte struct, same layout as the reference:
 * vendorId@0 (0x1002), deviceId@4 (PCI device id), dedicatedVRAM@8,
 * sharedMemory@16 (0), isIntegrated@24, description[128]@28. */
typedef struct GPUInfo {
  uint32_t vendorId;
  uint32_t deviceId;
  uint64_t dedicatedVRAM;
  uint64_t sharedMemory;
  uint32_t isIntegrated;
  char description[128];
} GPUInfo;
void GetGPUInfo(GPUInfo* info);

/* --------------------------------------------------------------- buffers -- */

/* engine.cpp:201 CreateBuffer.  refcount 1, taken from a size-keyed pool when
 * possible, so contents are stale when data == NULL.  `data` (count floats)
 * is consumed before return; the copy to the device is queued on the stream.
 * NULL on failure (count == 0 included). */
void* CreateBuffer(float* data, uint32_t count);
/* engine.cpp:255 AddRefBuffer. */
void AddRefBuffer(void* handle);
/* engine.cpp:284 ReleaseBuffer.  --refcount; at zero the buffer returns to the
 * pool (or is freed).  NULL is a no-op; a released handle is rejected. */
void ReleaseBuffer(void* handle);
/* engine.cpp:676 ReleaseBufferBatch. */
void ReleaseBufferBatch(void** handles, uint32_t count);
/* engine.cpp:261 UpdateBuffer: overwrite the whole buffer from host memory. */
void UpdateBuffer(void* handle, float* data);
/* engine.cpp:292 ReadBuffer: blocking; waits for all queued work, copies the
 * full buffer to dst. */
void ReadBuffer(void* handle, float* dst);
/* engine.cpp:349 ClearBuffer: zero all bits (a fill kernel, queued). */
void ClearBuffer(void* handle);
/* engine.cpp:325 FlushGPU: no-op (HIP submits at launch). */
void FlushGPU(void);
/* engine.cpp:331 SyncGPU: wait until the engine stream is idle. */
void SyncGPU(void);

/* engine.cpp:617 WarmPool, :637 GetPoolStats, :642 ResetPoolStats,
 * :648 GetPoolMemory, :653 DrainPool -- same meaning. */
void WarmPool(uint32_t* sizes, uint32_t numSizes, uint32_t copies);
void GetPoolStats(uint64_t* hits, uint64_t* misses);
void ResetPoolStats(void);
uint64_t GetPoolMemory(void);
void DrainPool(void);

/* -------------------------------------------------------------- dispatch -- */

/* engine.cpp:136 CompileShader.  No HLSL is compiled: returns true when `name`
 * is a kernel this library implements (path ignored), false otherwise. */
bool CompileShader(const char* name, const wchar_t* path);
/* engine.cpp:154 CompileShaderEx.  Custom HLSL is not supported: false. */
bool CompileShaderEx(const char* name, const wchar_t* path, const char* entry);

/* engine.cpp:396 RunShader / :404 RunShaderRaw.  Runs kernel `name` with
 * inputs srvs[0..nS) (HLSL t-registers), outputs uavs[0..nU) (u-registers)
 * and the packed 4-byte constant-buffer fields `cb` of the reference shader
 * of that name.  `threads` (D3D group counts) is accepted and ignored: the
 * launch shape is derived from the constants.  Reads outside a buffer return
 * 0 and writes outside it are dropped, as with D3D11 structured buffers.
 * Unknown names do nothing (as the reference) and set the last error. */
void RunShader(const char* name, void** srvs, uint32_t srvCount, void** uavs,
               uint32_t uavCount, uint32_t* threads, void* cb, uint32_t cbSize);
void RunShaderRaw(const char* name, void** srvs, uint32_t srvCount, void** uavs,
                  uint32_t uavCount, uint32_t* threads, void* cb, uint32_t cbSize);
/* engine.cpp:409 RunShaderAlloc / :419 RunShaderAlloc2. */
void* RunShaderAlloc(const char* name, void** srvs, uint32_t srvCount, uint32_t outCount,
                     uint32_t* threads, void* cb, uint32_t cbSize);
void* RunShaderAlloc2(const char* name, void** srvs, uint32_t srvCount, uint32_t outCount,
                      void* extraUav, uint32_t* threads, void* cb, uint32_t cbSize);

/* engine.cpp:934 ResolveShader, :952 RunSequence, :969 RunSequenceWithSGD.
 * SeqCmd is the reference's 200-byte record (shader@0, srvs[8]@8,
 * srvCount@72, uavs[4]@80, uavCount@112, threads[3]@116, cbData[64]@128,
 * cbSize@192); `shader` is a value returned by ResolveShader. */
typedef struct SeqCmd {
  void* shader;
  void* srvs[8];
  uint32_t srvCount;
  void* uavs[4];
  uint32_t uavCount;
  uint32_t threads[3];
  uint8_t cbData[64];
  uint32_t cbSize;
  uint32_t pad[1];
} SeqCmd;
void* ResolveShader(const char* name);
void RunSequence(SeqCmd* cmds, uint32_t count);
void RunSequenceWithSGD(SeqCmd* cmds, uint32_t cmdCount, void** params, void** grads,
                        uint32_t* sizes, uint32_t numParams, float lr, float clip);

/* --------------------------------------------------------- fused (hot path) */

/* engine.cpp:741 MatMulAlloc: C[M×N] = op(A)·op(B); flags bit0: A stored K×M,
 * bit1: B stored N×K.  fp32 MFMA GEMM.  NULL if A or B is smaller than the
 * shape implies (the reference would read zeros). */
void* MatMulAlloc(void* a, void* b, uint32_t M, uint32_t K, uint32_t N, uint32_t flags);

/* engine.cpp:751 ConvForwardFused: y = act(conv(x, W) + b), NCHW, act 0 id,
 * 1 ReLU, 2 tanh.  Implicit GEMM: no im2col matrix exists.  When pIm2col !=
 * NULL, *pIm2col receives the channel-innermost copy of x (padded to a
 * multiple of 4 channels, the size of x) that the forward built; it is an
 * opaque handle that ConvBackwardFused consumes, as the reference's im2col
 * buffer.  Operands of 2 GiB or more are refused (NULL + error). */
void* ConvForwardFused(void* x, void* filters, void* bias, uint32_t batch, uint32_t inC,
                       uint32_t inH, uint32_t inW, uint32_t outC, uint32_t kH, uint32_t kW,
                       uint32_t stride, uint32_t padding, uint32_t actType, void** pIm2col);

/* engine.cpp:802 ConvBackwardFused: G = dy masked by (y > 0) when actType == 1
 * and y != NULL (act 2 applies no derivative, as the reference); dW = G·colᵀ,
 * db = Σ G, dX = col2im(Wᵀ·G), each only when requested (NULL otherwise).
 * Consumes (releases) the im2col handle, as the reference; with im2col ==
 * NULL the channel-innermost copy of x is rebuilt from x.  dW/dX are
 * implicit-GEMM fp32 MFMA kernels; db is reduced from partials written by the
 * pass that masks and transposes dy into G. */
void ConvBackwardFused(void* gradOut, void* fwdOut, void* x, void* filters, void* im2col,
                       uint32_t batch, uint32_t inC, uint32_t inH, uint32_t inW,
                       uint32_t outC, uint32_t kH, uint32_t kW, uint32_t stride,
                       uint32_t padding, uint32_t actType, uint32_t xReq, uint32_t wReq,
                       uint32_t bReq, void** pDFilters, void** pDBias, void** pDInput);

/* engine.cpp:881 MaxPoolForwardFused: strict '>' window scan, absolute flat
 * input index stored as u32 bits in a float buffer (*pIndices). */
void* MaxPoolForwardFused(void* x, uint32_t batch, uint32_t inC, uint32_t inH, uint32_t inW,
                          uint32_t poolSize, uint32_t stride, void** pIndices);

/* engine.cpp:906 MaxPoolBackwardFused: dX routed through the indices and
 * consumes (releases) them.  Overlapping windows SUM their contributions
 * deterministically (the reference's store races). */
void* MaxPoolBackwardFused(void* gradOut, void* indices, uint32_t batch, uint32_t inC,
                           uint32_t outH, uint32_t outW, uint32_t xSize);

/* engine.cpp:436 SGDBatch: w -= lr*clamp(g, -clip, clip) for every non-NULL
 * (param, grad) pair; one multi-tensor launch. */
void SGDBatch(void** params, void** grads, uint32_t* sizes, uint32_t numParams, float lr,
              float clip);
/* engine.cpp:494 SGDBatchClipped: global-norm clip then SGD; blocking, returns
 * the norm. */
float SGDBatchClipped(void** params, void** grads, uint32_t* sizes, uint32_t numParams,
                      float lr, float maxNorm);

/* ------------------------------------------------------------- additions --
 * Entry points with no engine.dll counterpart.  They give the host layer
 * single-launch versions of loops the reference runs from Python. */

/* Reason for the last failure ("" if none). */
const char* GetLastErrorString(void);
void ClearLastError(void);

/* One multi-tensor launch of the reference's per-parameter `adam` dispatches
 * (AdamW.step, nn_engine.py:2217-2238; nn_adam.hlsl:20-33): element clip,
 * moments, w -= wd*w + step*m/(sqrt(v)+eps).  NULL params/grads are skipped. */
void AdamBatch(void** params, void** grads, void** m, void** v, uint32_t* sizes,
               uint32_t numParams, float stepSize, float beta1, float beta2, float eps,
               float weightDecay, float clip);

/* GPU form of clip_grad_norm (nn_engine.py:1335-1355): norm = sqrt(sum g^2)
 * over all grads; when norm > maxNorm every grad is scaled in place by
 * maxNorm/(norm+1e-6).  Blocking; returns the norm. */
float ClipGradNorm(void** grads, uint32_t* sizes, uint32_t numGrads, float maxNorm);

/* AdamBatch with the step counter kept on the device, so that a recorded
 * step (BeginCapture) replays as the next step, not as a copy of the recorded
 * one.  stepState is a buffer of at least 2 floats: [0] = t (u32 bits),
 * [1] = the step size lr*sqrt(1-beta2^t)/(1-beta1^t) of that step.  t > 0
 * sets the counter to t and the step size to stepSize, which the caller
 * evaluates as AdamW.step does in Python (nn_engine.py:2217-2238).  t == 0
 * advances the counter by one and evaluates the step size on the device, in
 * double from the double hyper-parameters, rounded once to float (use 0 in a
 * recorded step; stepSize is then ignored).  weightDecay is lr*wd, as
 * AdamBatch. */
void AdamBatchCounted(void** params, void** grads, void** m, void** v, uint32_t* sizes,
                      uint32_t numParams, void* stepState, uint32_t t, float stepSize,
                      double lr, double beta1, double beta2, float eps, float weightDecay,
                      float clip);

/* ClipGradNorm that allocates nothing.  It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same kernels, arguments and result as ClipGradNorm, but the partial sums
 * live in a static device array of 65536 doubles (512 KiB, held by every GPU
 * the library runs on until the process ends) instead of the growable
 * workspace: at most 65536 chunks of 4096 gradient elements (268,435,456
 * elements when every tensor fills its chunks; each tensor rounds up to whole
 * chunks).  Larger requests are refused: returns -1 and sets the error.
 * Calls on one GPU share its array, so calls that overlap on one GPU race;
 * the library's single stream keeps its own calls in order.  Blocking;
 * returns the norm (NaN while a capture is open). */
float ClipGradNormNoAlloc(void** grads, uint32_t* sizes, uint32_t numGrads, float maxNorm);

/* Kernel-family timing with HIP events on the engine stream (for bench.py).
 * SetProfiling(1) starts recording every launch of the named families;
 * GetProfile returns launches, summed milliseconds, summed algorithmic
 * FLOPs and bytes for one family ("conv_dw", "conv_dx", "conv_fwd", "gemm",
 * ...) and returns false for an unknown family. */
void SetProfiling(int enabled);
bool GetProfile(const char* family, uint64_t* launches, double* ms, double* flops,
                double* bytes);
void ResetProfile(void);
/* Restrict recording to a comma-separated list of families (NULL or "": all),
 * so that a timed run carries only the events it reports. */
void SetProfileFilter(const char* families);

/* One HIP-event pair around all work queued between the two calls, recorded
 * as one launch of `family` with the given algorithmic FLOPs and bytes
 * (GetProfile reads it back), independent of SetProfiling.  For timing a
 * run of back-to-back launches without an event pair per launch.  One region
 * at a time; refused while capturing. */
bool BeginProfileRegion(const char* family, double flops, double bytes);
bool EndProfileRegion(void);

/* Passes that move more than `bytes` bytes use nontemporal (streaming) loads
 * and stores; smaller ones use the default cache policy.  The default is
 * 256 MiB, the size of the MI355X Infinity Cache; a negative value restores
 * it.  Returns the previous threshold.  The choice changes speed only, never
 * results: it exists for tuning and so that tests can run both kernel forms
 * at small sizes. */
double SetStreamingThreshold(double bytes);

/* Record / replay of queued work as a HIP graph: the MI355X form of the
 * reference's ComputeGraph (nn_engine.py:2505-2771), which records RunShader
 * dispatches and replays them through RunSequence (engine.cpp:952).  Between
 * BeginCapture and EndCapture every launch on the engine stream is captured
 * instead of run -- the fused conv / pool / matmul calls included -- and every
 * buffer handed out is held until ReleaseGraph.  Calls that wait on the
 * stream (ReadBuffer, SyncGPU, ReplayGraph, ReleaseGraph) and host uploads of
 * more than 256 floats are refused while capturing; EndCapture then returns
 * NULL with the reason in GetLastErrorString.  ClipGradNorm and
 * SGDBatchClipped return NaN while capturing (the norm exists only when the
 * graph runs).  ReplayGraph enqueues one replay; kernel arguments (sizes,
 * host scalars, small uploads) are those of the captured call. */
bool BeginCapture(void);
void* EndCapture(void);
bool ReplayGraph(void* graph);
void ReleaseGraph(void* graph);

#ifdef __cplusplus
}
#endif
#endif /* DCENGINE_H */
