// sinkattn_block_sparse_attn_noalloc: the block-sparse forward from a bool mask for callers
// that cannot allocate device memory.  It is sinkattn_block_sparse_plan followed by
// sinkattn_block_sparse_fwd (the same validation, kernels and results), with the plan held
// in `scratch`, a library-owned static device array, instead of caller buffers.
//
// Host code never uses the array's name as an address (on the host it is only a stand-in
// symbol): the device address is looked up once per GPU with hipGetSymbolAddress, with that
// GPU current, and only that pointer is handed to the kernels.  The plan kernels write every
// entry the forward reads (counts, the listed prefix of each idx row, every order slot), so
// nothing has to be cleared between calls.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "../../include/sinkattn.h"
#include "kernels.h"

// Plan of the last call on this GPU: counts | order | idx, each 256-byte aligned.  Every
// GPU the library runs on holds its own copy until the process ends.
static __device__ __align__(256) unsigned char scratch[SINKATTN_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;

std::mutex g_lookup_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

int64_t align256(int64_t bytes) { return (bytes + 255) / 256 * 256; }

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Device address of the current GPU's copy of `scratch`, looked up on the first call per
// GPU.  That lookup may load the library's code object on the GPU, which must not happen
// while `stream` is being captured into a graph: an uncached first call under capture is
// refused (*refused = true, nothing looked up), so callers make one call outside capture
// first.
hipError_t scratch_on_current_device(hipStream_t stream, void** out, bool* refused) {
  *refused = false;
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_lookup_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cs);
    if (e != hipSuccess) return e;
    if (cs != hipStreamCaptureStatusNone) {
      *refused = true;
      return hipSuccess;
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

}  // namespace

extern "C" int sinkattn_block_sparse_attn_noalloc(
    const uint8_t* mask, const int64_t mask_strides[4], const void* q, const void* k,
    const void* v, int dtype, int64_t B, int64_t H, int64_t Nq, int64_t Nk, int64_t D,
    const int64_t q_strides[4], const int64_t k_strides[4], const int64_t v_strides[4], void* out,
    const int64_t out_strides[4], float* lse, float softmax_scale, void* stream) {
  if (B < 0 || H < 0 || Nq < 0 || Nk < 0) return sa::api_fail("attn_noalloc: negative size");
  const int64_t nqb = cdiv(Nq, 128), nkb = cdiv(Nk, 128);
  if (B * H * nqb == 0) return 0;
  if (nkb > 8192) return sa::api_fail("attn_noalloc: %lld key blocks (at most 8192)", (long long)nkb);
  const int64_t rows = B * H * nqb;
  // the plan, in bytes: counts + order slots + index lists, each 256-byte aligned
  const int64_t cap = (int64_t)SINKATTN_NOALLOC_SCRATCH_BYTES;
  if (rows > cap / 4 / (nkb + 1))
    return sa::api_fail("attn_noalloc: B*H*nqb*nkb = %lld mask entries need more than the %lld-byte "
                        "static plan buffer; use sinkattn_block_sparse_plan + sinkattn_block_sparse_fwd",
                        (long long)(rows * nkb), (long long)cap);
  const int64_t slots = sinkattn_block_sparse_order_slots(B, H, nqb);
  const int64_t counts_bytes = align256(rows * 4);
  const int64_t order_bytes = align256(slots * 4);
  const int64_t idx_bytes = align256(rows * nkb * 4);
  if (slots <= 0 || counts_bytes + order_bytes + idx_bytes > cap)
    return sa::api_fail("attn_noalloc: the plan needs %lld bytes, more than the %lld-byte static "
                        "plan buffer; use sinkattn_block_sparse_plan + sinkattn_block_sparse_fwd",
                        (long long)(counts_bytes + order_bytes + idx_bytes), (long long)cap);
  void* base = nullptr;
  bool refused = false;
  const int st = sa::api_hip_status(scratch_on_current_device(static_cast<hipStream_t>(stream), &base, &refused),
                                    "attn_noalloc: plan buffer address");
  if (st != 0) return st;
  if (refused)
    return sa::api_fail("attn_noalloc: the first call on a GPU looks up the static plan buffer's address and "
                        "must not run under stream capture; make one call outside capture first");
  unsigned char* p = static_cast<unsigned char*>(base);
  int32_t* counts = reinterpret_cast<int32_t*>(p);
  int32_t* order = reinterpret_cast<int32_t*>(p + counts_bytes);
  int32_t* idx = reinterpret_cast<int32_t*>(p + counts_bytes + order_bytes);
  const int rc = sinkattn_block_sparse_plan(mask, mask_strides, B, H, nqb, nkb, counts, idx, order, stream);
  if (rc != 0) return rc;
  return sinkattn_block_sparse_fwd(q, k, v, dtype, B, H, Nq, Nk, D, q_strides, k_strides, v_strides,
                                   out, out_strides, lse, counts, idx, order, nqb, nkb,
                                   softmax_scale, stream);
}
