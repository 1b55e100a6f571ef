// One call per Int8Linear layer: the quantizer (with the low-rank down-projection when the layer has one) and the
// fused GEMM, with the codes, row scales and t staged in a workspace between the two kernels
// (reference: Int8Linear.forward, deploy/int8_exec.py:382-393).
//
// Workspace layout for M rows, K inputs and R columns of t (offsets rounded up to 256 bytes):
//   [0, QB)           packed K64 codes, QB = ceil(M / 16) * 16 * K bytes
//   [SO, SO + 4 M)    fp32 row scales, SO = round256(QB)
//   [TO, TO + 2 M R)  16-bit t [M, R], TO = SO + round256(4 M)
//   [CO, CO + 36)     the GEMM's scheduling buffer (9 int32 claim counters), CO = TO + round256(2 M R)
// The quantizer writes every byte the GEMM reads (padding code rows included) and zeroes the scheduling buffer in
// the same kernel, so the workspace needs no clearing and may hold anything on entry.
#include "pq_common.h"

#include <mutex>

namespace pq {
namespace {

constexpr int64_t round256(int64_t b) { return (b + 255) & ~int64_t(255); }

struct LayerSlices {
  int64_t scales, t, sched, total;
};

constexpr int64_t kSchedBytes = 9 * sizeof(int32_t);

LayerSlices layer_slices(int64_t M, int64_t K, int64_t R) {
  LayerSlices s;
  s.scales = round256(((M + 15) / 16) * 16 * K);
  s.t = s.scales + round256(4 * M);
  s.sched = s.t + round256(2 * M * R);
  s.total = s.sched + kSchedBytes;
  return s;
}

}  // namespace

// The layer over a workspace the caller provides (shared by pq_int8_linear and its allocation-free variant).
static int run_layer(const void* x, int32_t x_dtype, int64_t M, int64_t K, int64_t ldx, const int8_t* w_packed,
                     const float* s_w, int64_t group, const float* bias, const void* l1t, const void* l1f, int64_t R,
                     const void* l2t, int64_t Re, void* y, int64_t ldy, int64_t N, uint8_t* ws, hipStream_t stream) {
  const LayerSlices sl = layer_slices(M, K, R);
  int8_t* const q = reinterpret_cast<int8_t*>(ws);
  float* const s = reinterpret_cast<float*>(ws + sl.scales);
  void* const t = R ? static_cast<void*>(ws + sl.t) : nullptr;
  int32_t* const sched = reinterpret_cast<int32_t*>(ws + sl.sched);   // zeroed by the quantizer kernel
  int st = R ? quant_rows_lowrank_z(x, x_dtype, M, K, ldx, M, nullptr, l1t, l1f, R, q, s, t, R, sched, stream)
             : quant_rows_packed_z(x, x_dtype, M, K, ldx, M, nullptr, q, s, sched, stream);
  if (st != PQ_OK) return st;
  return int8_gemm_packed(q, w_packed, s, s_w, group, bias, R ? t : nullptr, R, R ? l2t : nullptr, Re, x_dtype, y, ldy,
                          x_dtype, nullptr, 0, M, N, K, sched, stream);
}

int check_layer(int64_t M, int64_t K, int64_t N, int64_t R, int64_t Re, const void* l1t, const void* l2t,
                const char* who) {
  if (M < 0 || K < 64 || N < 64) return set_error(PQ_ESHAPE, "%s: bad shape M=%lld K=%lld N=%lld", who, (long long)M, (long long)K, (long long)N);
  if (K % 64 || N % 64) return set_error(PQ_ESHAPE, "%s: need K %% 64 == 0 and N %% 64 == 0", who);
  if (R < 0 || Re < 0 || (R == 0) != (Re == 0) || (R && (!l1t || !l2t)))
    return set_error(PQ_EINVAL, "%s: a low-rank branch needs l1t, l2t and both ranks (R=%lld, Re=%lld)", who,
                     (long long)R, (long long)Re);
  if (R && Re > R) return set_error(PQ_ESHAPE, "%s: epilogue rank %lld exceeds the %lld columns of t", who, (long long)Re, (long long)R);
  return PQ_OK;
}

}  // namespace pq

using namespace pq;

extern "C" int64_t pq_int8_linear_workspace_size(int64_t M, int64_t K, int64_t R) {
  if (M < 0 || K < 1 || R < 0) return -1;
  return layer_slices(M, K, R).total;
}

extern "C" int pq_int8_linear(const void* x, int32_t x_dtype, int64_t M, int64_t K, int64_t ldx,
                              const int8_t* w_packed, const float* s_w, int64_t group, const float* bias,
                              const void* l1t, const void* l1f, int64_t R, const void* l2t, int64_t Re, void* y,
                              int64_t ldy, int64_t N,
                              void* workspace, int64_t ws_bytes, hipStream_t stream) {
  int st = check_layer(M, K, N, R, Re, l1t, l2t, "pq_int8_linear");
  if (st != PQ_OK || M == 0) return st;
  const int64_t need = layer_slices(M, K, R).total;
  if (!workspace || ws_bytes < need)
    return set_error(PQ_ESHAPE, "pq_int8_linear: the workspace holds %lld bytes, the layer needs %lld", (long long)ws_bytes,
                     (long long)need);
  if ((uintptr_t)workspace % 256) return set_error(PQ_EALIGN, "pq_int8_linear: the workspace must be 256-byte aligned");
  return run_layer(x, x_dtype, M, K, ldx, w_packed, s_w, group, bias, l1t, l1f, R, l2t, Re, y, ldy, N,
                   static_cast<uint8_t*>(workspace), stream);
}

// ---- allocation-free variant -------------------------------------------------------------------------------------
// For callers that cannot allocate device memory (code under HIP graph capture, serving loops, harnesses that forbid
// hipMalloc): the workspace is this file-scope device array, one copy per GPU, held until the process ends. In host
// code `scratch` names a host-side stand-in, not the device array: its device address comes from
// hipGetSymbolAddress, once per device (with that device current), and only that address is passed to kernels.
// Every call on a GPU shares that GPU's array, so calls that overlap on one GPU (two streams, two threads) race.
// Nothing here needs clearing: the quantizer writes every byte of the slices the GEMM reads, and zeroes the GEMM's
// scheduling buffer (the array's workspace layout is pq_int8_linear's).
constexpr int64_t kScratchBytes = 64LL << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[kMaxDevices] = {};   // device address of `scratch` on each device, once looked up

// Device address of this device's scratch array; the stream must belong to the current device.
int device_scratch(hipStream_t stream, uint8_t** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(PQ_ELAUNCH, "pq_int8_linear_noalloc: no usable current device");
  if (stream) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess)
      return set_error(PQ_EINVAL, "pq_int8_linear_noalloc: cannot query the stream's device");
    if (sdev != dev)
      return set_error(PQ_EINVAL, "pq_int8_linear_noalloc: the stream belongs to device %d, device %d is current",
                       (int)sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(PQ_ELAUNCH, "pq_int8_linear_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<uint8_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return PQ_OK;
}
}  // namespace

extern "C" int64_t pq_int8_linear_noalloc_max_bytes(void) { return kScratchBytes; }

extern "C" int pq_int8_linear_noalloc(const void* x, int32_t x_dtype, int64_t M, int64_t K, int64_t ldx,
                                      const int8_t* w_packed, const float* s_w, int64_t group, const float* bias,
                                      const void* l1t, const void* l1f, int64_t R, const void* l2t, int64_t Re,
                                      void* y, int64_t ldy,
                                      int64_t N, hipStream_t stream) {
  int st = check_layer(M, K, N, R, Re, l1t, l2t, "pq_int8_linear_noalloc");
  if (st != PQ_OK || M == 0) return st;
  const int64_t need = layer_slices(M, K, R).total;
  if (need > kScratchBytes)
    return set_error(PQ_ESHAPE,
                     "pq_int8_linear_noalloc: M=%lld, K=%lld, R=%lld needs %lld bytes of staging, more than the %lld "
                     "bytes of its device scratch; use pq_int8_linear with a workspace",
                     (long long)M, (long long)K, (long long)R, (long long)need, (long long)kScratchBytes);
  uint8_t* ws = nullptr;
  st = device_scratch(stream, &ws);
  if (st != PQ_OK) return st;
  return run_layer(x, x_dtype, M, K, ldx, w_packed, s_w, group, bias, l1t, l1f, R, l2t, Re, y, ldy, N, ws, stream);
}
