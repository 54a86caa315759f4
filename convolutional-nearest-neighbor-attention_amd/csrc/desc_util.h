// Descriptor-derived sizes shared by the C-ABI translation units.
#pragma once

#include <math.h>
#include <stdint.h>

#include "common.h"
#include "kernels.h"

namespace cnna_desc_util {

inline int elem_size(int dtype) {
  return (dtype == CNNA_BF16 || dtype == CNNA_F16) ? 2 : (dtype == CNNA_F32 ? 4 : 0);
}

inline int din_of(const cnna_desc* d) { return d->C / d->H + (d->coord ? 1 : 0); }

// channels padded to the MFMA reduction depth (16) and 16-byte rows
inline int dkp_of(const cnna_desc* d) { return (int)cnna_round_up((size_t)din_of(d), 16); }

inline int ksel_of(const cnna_desc* d) { return d->sampled ? d->K - 1 : d->K; }

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// matmul similarity scale: the descriptor's, else 1/sqrt(d_k) (layers.py:324)
inline float matmul_scale(const cnna_desc* d) {
  return d->scale != 0.0f ? d->scale : (float)(1.0 / sqrt((double)(d->C / d->H)));
}

// aggregate-kernel layout of z for the descriptor's cnna_merge
inline int merge_mode(const cnna_desc* d) {
  return d->merge == CNNA_MERGE_CONCAT ? MERGE_CONCAT : MERGE_REFERENCE;
}

// bump allocator over a caller workspace (256-byte aligned slices)
struct Carve {
  char* p;
  size_t used = 0;
  explicit Carve(void* base) : p(static_cast<char*>(base)) {}
  void* take(size_t bytes) {
    void* r = p ? p + used : nullptr;
    used += cnna_round_up(bytes, 256);
    return r;
  }
};

}  // namespace cnna_desc_util
