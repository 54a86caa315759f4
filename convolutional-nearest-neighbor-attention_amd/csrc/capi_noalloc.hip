// cnna_forward_noalloc: the whole forward (cnna_forward) for callers that
// cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc).  Its intermediates live in a
// file-scope device array of CNNA_NOALLOC_SCRATCH_BYTES instead of a caller
// workspace.
//
// The array's name is a host-side stand-in, not a device address: its address
// on a device is looked up once per device with hipGetSymbolAddress (with that
// device current) and only that pointer is handed to the kernels.  Each GPU
// holds its own copy of the array from the first call until the process ends.
// Calls on one GPU share it: calls that overlap on one GPU (concurrent streams
// or threads) race, and each call leaves its intermediates there.  None of the
// forward kernels reads scratch memory it has not written in the same call,
// so nothing needs clearing between calls.
#include <mutex>

#include "common.h"
#include "kernels.h"

#include "desc_util.h"

namespace {

static __device__ __align__(256) unsigned char scratch[CNNA_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void* g_ptr[MAX_DEVICES] = {};

// device address of `scratch` on the current device (looked up once per device)
int scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= MAX_DEVICES) return CNNA_ERR_SHAPE;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (p == nullptr) return (int)hipErrorInvalidSymbol;
    g_ptr[dev] = p;
  }
  *out = g_ptr[dev];
  return CNNA_OK;
}

}  // namespace

extern "C" {

int cnna_forward_noalloc(const cnna_desc* d, const void* x, int64_t ldx, const int32_t* cand,
                         const void* Wq, const void* Wk, const void* Wv, const void* Wo,
                         const void* conv_w0, const void* conv_w1, void* out, int64_t ldo,
                         void* stream) {
  int st = cnna_check_desc(d);
  if (st) return st;
  const size_t need = cnna_forward_workspace(d);
  if (need > (size_t)CNNA_NOALLOC_SCRATCH_BYTES) return CNNA_ERR_SCRATCH;
  void* ws = nullptr;
  if ((st = scratch_ptr(&ws))) return st;
  return cnna_forward(d, x, ldx, cand, Wq, Wk, Wv, Wo, conv_w0, conv_w1, out, ldo, ws,
                      (size_t)CNNA_NOALLOC_SCRATCH_BYTES, stream);
}

}  // extern "C"
