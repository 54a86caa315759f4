// Implementation of the fused similarity + streaming top-k kernel; included by
// select_{bf16,f16,f32}{,_euc}.hip so that the dtypes and the euclidean
// instances compile in parallel.
//
// Replaces layers.py:323-340 followed by torch.topk in layers.py:344, 363,
// 391, 410 and the sampled self mask layers.py:291-292, 304-305.  The N x Nq
// similarity never reaches HBM.
//
// Block = 4 waves; a wave owns 32 tokens of one (batch, head).  Candidate
// (query) tiles of TJ = 32 rows are staged through LDS, double buffered, and
// each wave computes S^T for its tokens with v_mfma_f32_32x32x{16 bf16|2 f32}:
// the A operand is the candidate tile and the B operand the wave's 32 key rows
// (kept in registers), so lane l holds 16 candidates of token l % 32 per tile;
// lanes l and l + 32 split a token's candidates.  The small tile keeps the
// register and LDS footprint low enough for three blocks per CU at d_k = 128.
//
// Ranking key (larger is better):
//   matmul / cosine, sampling 'all': the raw accumulator k.q (the positive
//     scale 1/sqrt(d_k) is applied to the selected values only; a negative
//     scale negates the key rows once, so the key is -k.q);
//   sampled paths: acc * kscale, with the self-masked candidate set to the
//     reference's constant;
//   euclidean: -d^2, d^2 = (|k|^2 + |q|^2) - 2 acc; a negative d^2 (NaN
//     distance in the reference) ranks last.
// Ties break by the lowest candidate index.
//
// Two passes over the candidates:
//  1. per lane, the maximum of each 16-candidate group (4-candidate groups
//     when Nq <= 512; rows of more than 16 tiles sweep only their first three
//     quarters, their first quarter for d >= 256 and at least 64 tiles) goes into a sorted
//     register list (med3 insertion); the K-th largest of the union of both
//     half-lanes' lists is a lower bound tau of the token's K-th key, because
//     it is attained by K distinct candidates.
//  2. the tiles are recomputed and every key >= tau is appended to a per-lane
//     LDS queue (about K + few entries per token).  When a queue fills, and at
//     the end, each half-lane sorts its queue into a list and the lower half
//     merges the two into the token's one sorted (key, index) list in LDS
//     (a bitonic top-K merge); tau then rises to just
//     above the list's K-th key for both halves.  Drains happen at tile
//     positions where both halves have consumed a prefix of the candidate
//     indices, so a later candidate never ties its way in ahead of a listed
//     one.  The list is written out with the neighbour weights.
//
// K wider than one list (KMAX = 32): rounds of at most 32 entries.  Round r
// (EX) excludes every candidate that ranks at or before the last entry of
// round r - 1 (compared as packed (key, index) pairs, so ties continue in index
// order); that entry is handed over in the idx / vals slot round r fills first.
// Pass 1 masks keys >= the excluded key (a superset, so tau stays a lower
// bound).  The weights of all K entries are computed by a final row kernel.
#pragma once
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace {

constexpr int TJ = 32;      // candidates per tile (one 32-row MFMA block)
constexpr int NB = TJ / 32; // MFMA blocks per tile
constexpr int TPB = 128;    // tokens per block
constexpr int QCMIN = 12;
constexpr int QCHK = 4;     // elements between queue checks
constexpr int NT = 256;     // threads per block

template <typename T> struct SelCfg;
// MAXCH: chunks of the regular instances; WIDECH: chunks of the wide-head
// instances (key rows of 128 registers per lane, one block per CU)
template <> struct SelCfg<uint16_t> { static constexpr int MAXCH = 16, WIDECH = 16, VEC = 8; };  // d <= 256
template <> struct SelCfg<_Float16> { static constexpr int MAXCH = 16, WIDECH = 16, VEC = 8; };  // d <= 256
template <> struct SelCfg<float> { static constexpr int MAXCH = 64, WIDECH = 128, VEC = 4; };    // d <= 128, wide 256

// A (key, index) pair as one 64-bit integer ordered like the ranking (larger
// key first, then lower index): high word = order-preserving image of the float key, low word = ~index.
// 0 (below every real entry) marks an empty list slot.
CNNA_DEV uint32_t ord_key(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
CNNA_DEV float key_of_ord(uint32_t u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}
CNNA_DEV uint64_t pack_entry(float key, uint32_t j) {
  return ((uint64_t)ord_key(key) << 32) | (uint64_t)(~j);
}

// insert x into the descending list L (one 64-bit compare per slot)
template <int KMAX>
CNNA_DEV void list_insert(uint64_t (&L)[KMAX], uint64_t x) {
  bool b[KMAX];
#pragma unroll
  for (int r = 0; r < KMAX; ++r) b[r] = x > L[r];
#pragma unroll
  for (int r = KMAX - 1; r >= 1; --r) L[r] = b[r - 1] ? L[r - 1] : (b[r] ? x : L[r]);
  L[0] = b[0] ? x : L[0];
}

// max(a, b) for non-NaN inputs as one VALU op (fmaxf, and a med3 against
// +inf, which the compiler turns into fmaxf, first canonicalise both operands:
// two more VALU ops)
CNNA_DEV float max2(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// max of three non-NaN floats, one VALU op
CNNA_DEV float max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

template <int KMAX>
CNNA_DEV void bound_insert(float (&L)[KMAX], float x) {
#pragma unroll
  for (int r = KMAX - 1; r >= 1; --r) L[r] = __builtin_amdgcn_fmed3f(L[r - 1], x, L[r]);
  L[0] = max2(L[0], x);
}

// L[r] for a runtime (wave-uniform) r, written as masked ORs so the
// compiler keeps the list in registers instead of indexing scratch memory.
template <int KMAX>
CNNA_DEV int pick(const int (&L)[KMAX], int r) {
  int t = 0;
#pragma unroll
  for (int i = 0; i < KMAX; ++i) t |= L[i] & -(int)(i == r);
  return t;
}
template <int KMAX>
CNNA_DEV uint64_t pick(const uint64_t (&L)[KMAX], int r) {
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < KMAX; ++i) {
    const uint32_t m = -(uint32_t)(i == r);
    lo |= (uint32_t)L[i] & m;
    hi |= (uint32_t)(L[i] >> 32) & m;
  }
  return ((uint64_t)hi << 32) | lo;
}
template <int KMAX>
CNNA_DEV float pick(const float (&L)[KMAX], int r) {
  int t = 0;
#pragma unroll
  for (int i = 0; i < KMAX; ++i) t |= __float_as_int(L[i]) & -(int)(i == r);
  return __int_as_float(t);
}

// NCH: number of MFMA reduction chunks (d / KC); EXACT: the head width equals
// NCH * KC (no per-chunk guards), otherwise NCH is an upper bound.
// Three or two blocks per CU where the register footprint allows it without spills.
// KFR: registers per lane holding the key rows (NCH fragments).
template <int KFR, int KMAX, bool EUC, bool SMP>
constexpr int sel_min_blocks() {
  return (KMAX <= 9 && KFR <= 32 && !EUC && !SMP) ? 3
         : (KMAX <= 16 && (KFR <= 32 || (KFR <= 64 && !EUC && !SMP)) &&
            ((!EUC && !SMP) || KFR * KMAX <= 288)) ? 2 : 1;
}

// Queue capacity per lane (drained when a lane passes QC - QCHK; block-wide
// drains at tile boundaries when any lane holds more than QC - 6).  An entry
// is 6 bytes (key bits, 16-bit candidate index; Nq <= 65536); the capacity is
// the largest of 20 / 16 / 12 slots whose LDS footprint still allows the
// instance's blocks per CU: more slots, fewer drains.
template <typename T, int NCH, bool EXACT, int KMAX, bool EUC, bool SMP>
constexpr int queue_cap() {
  constexpr int VEC = SelCfg<T>::VEC;
  constexpr int dk = NCH * Mfma<T>::KC;
  constexpr int fixed = 2 * 32 * (dk + VEC) * (int)sizeof(T) + 2 * 32 * 8 + 32 + KMAX * 128 * 8;
  constexpr int budget = (160 * 1024) / sel_min_blocks<NCH * (sizeof(T) == 2 ? 4 : 1), KMAX, EUC, SMP>() - 1024;
  return !EXACT ? 12 : (fixed + 20 * 256 * 6 <= budget ? 20 : (fixed + 16 * 256 * 6 <= budget ? 16 : 12));
}

template <typename T, int NCH, bool EXACT, int KMAX, bool EUC, bool SMP, bool EX = false>
__global__ __launch_bounds__(NT, (sel_min_blocks<NCH * (sizeof(T) == 2 ? 4 : 1), KMAX, EUC, SMP>()))
void select_kernel(SelArgs a) {
  using M_ = Mfma<T>;
  constexpr int VEC = SelCfg<T>::VEC;
  constexpr bool RAW = !EUC && !SMP;     // keys are raw accumulators
  // short MFMA work per tile (d <= 128): predicated appends measured faster;
  // wider heads hide the branch-free stores behind the longer MFMA chain
  constexpr bool PRED_APPEND = NCH * Mfma<T>::KC <= 128;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int total = a.BH * a.rb_per_bh;
  const int w = xcd_swizzle(blockIdx.x, total);
  const int bh = w / a.rb_per_bh, rb = w - bh * a.rb_per_bh;
  const int ti = rb * TPB + wave * 32 + col;
  const bool tvalid = ti < a.N;
  const int tic = tvalid ? ti : a.N - 1;

  const int dkp = EXACT ? NCH * M_::KC : a.dkp;
  const int nch = dkp / M_::KC;
  const int QS = dkp + VEC;  // LDS row stride of a candidate tile (elements)
  T* qt = reinterpret_cast<T*>(smem);
  float* qnt = reinterpret_cast<float*>(smem + 2 * TJ * QS * sizeof(T));
  int* cdt = reinterpret_cast<int*>(qnt + 2 * TJ);
  constexpr int QC = queue_cap<T, NCH, EXACT, KMAX, EUC, SMP>();
  // queue: key bits [QC][NT] (32-bit) followed by candidate indices [QC][NT]
  // (16-bit); slot e of lane tid at qent[e * NT + tid] / qidx[e * NT + tid]
  int* dflag = cdt + 2 * TJ;   // [2][4] per-wave drain requests, by tile parity
  uint32_t* qent = reinterpret_cast<uint32_t*>(dflag + 8);

  const T* Kb = static_cast<const T*>(a.k) + ((int64_t)bh * a.N + tic) * dkp;
  const T* Qb = static_cast<const T*>(a.q) + (int64_t)bh * a.Nq * dkp;
  const float kni = EUC ? a.kn[(int64_t)bh * a.N + tic] : 0.0f;

  typename M_::frag kf[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c)
    kf[c] = (EXACT || c < nch) ? M_::load(Kb + c * M_::KC + half * M_::KL) : M_::zero();
  // a negative matmul scale ranks the smallest k.q first: rank on -k.q
  if (RAW && a.kneg) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) kf[c] = M_::neg(kf[c]);
  }
  // a later round: the previous round's last entry (key, candidate index)
  constexpr int OFF = SMP ? 1 : 0;
  float ekey = 0.0f;
  uint32_t ej = 0;
  if (EX) {
    const int64_t eo = ((int64_t)bh * a.N + tic) * a.K + OFF + a.kbase;
    ekey = key_of_ord(__float_as_uint(a.vals[eo]));
    ej = ~(uint32_t)a.idx[eo];
  }
  // wait for the key rows here, so the tile loop carries no vector-memory waits
  // ahead of its MFMAs (s_waitcnt vmcnt(0))
  __builtin_amdgcn_s_waitcnt(0x0F70);

  const int ntiles = (a.Nq + TJ - 1) / TJ;
  const int vpr = dkp / VEC;  // 16-byte vectors per candidate row
  constexpr int NPF = (TJ * (NCH * Mfma<T>::KC / VEC) + NT - 1) / NT;
  // every thread's NPF vectors lie inside the tile (narrow heads have fewer
  // vectors per tile than threads: the extra threads must not store)
  constexpr bool FULLV = EXACT && (TJ * (NCH * Mfma<T>::KC / VEC)) % NT == 0;

  // ---- tile staging: unconditional loads of clamped rows (rows >= Nq are
  // masked when keys are formed), so no load sits behind a branch
  // PD register sets: tile t+2 is loaded PD steps before it is stashed, which
  // covers the load latency when a step is short (narrow heads)
  constexpr int PD = NPF <= 1 ? 2 : 1;
  u32x4_t pfs[PD][NPF];
  float pfns[PD] = {};
  int pfcs[PD] = {};
  auto fetch = [&](int tile, auto SLOT) __attribute__((always_inline)) {
    u32x4_t (&pf)[NPF] = pfs[decltype(SLOT)::value];
    float& pfn = pfns[decltype(SLOT)::value];
    int& pfc = pfcs[decltype(SLOT)::value];
    __builtin_amdgcn_s_setprio(2);
    const int j0 = tile * TJ;
#pragma unroll
    for (int i = 0; i < NPF; ++i) {
      const int e = tid + i * NT;
      int r = e / vpr;
      const int cv = e - r * vpr;
      r = min(j0 + min(r, TJ - 1), a.Nq - 1);
      pf[i] = *reinterpret_cast<const u32x4_t*>(Qb + (int64_t)r * dkp + cv * VEC);
    }
    __builtin_amdgcn_s_setprio(0);
    if (EUC || SMP) {
      const int j = min(j0 + (tid & (TJ - 1)), a.Nq - 1);
      if (EUC) pfn = a.qn[(int64_t)bh * a.Nq + j];
      if (SMP) pfc = a.cand[j];
    }
  };
  auto stash = [&](int buf, auto SLOT) __attribute__((always_inline)) {
    const u32x4_t (&pf)[NPF] = pfs[decltype(SLOT)::value];
    const float pfn = pfns[decltype(SLOT)::value];
    const int pfc = pfcs[decltype(SLOT)::value];
    T* dst = qt + buf * TJ * QS;
#pragma unroll
    for (int i = 0; i < NPF; ++i) {
      const int e = tid + i * NT;
      const int r = e / vpr, cv = e - r * vpr;
      if (FULLV || r < TJ) *reinterpret_cast<u32x4_t*>(dst + r * QS + cv * VEC) = pf[i];
    }
    if (tid < TJ) {
      if (EUC) qnt[buf * TJ + tid] = pfn;
      if (SMP) cdt[buf * TJ + tid] = pfc;
    }
  };

  // S^T tile for this wave: acc[blk][v] = k_ti . q_{j0 + blk*32 + mfma_row(v)}
  auto compute = [&](int buf, f32x16_t (&acc)[NB]) __attribute__((always_inline)) {
    const T* base = qt + buf * TJ * QS + col * QS + half * M_::KL;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[b][v] = 0.0f;
    // the MFMA chain (and below, the next tile's global loads) is issued at a
    // raised wave priority, ahead of the other waves' filter work on the SIMD,
    // so the matrix core starts sooner (c3 select about 2 % faster)
    __builtin_amdgcn_s_setprio(2);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (EXACT || c < nch) {
        typename M_::frag af[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) af[b] = M_::load(base + b * 32 * QS + c * M_::KC);
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b] = M_::mma(af[b], kf[c], acc[b]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };
  // ranking key of one accumulator entry
  auto keyof = [&](float accv, int buf, int jl) __attribute__((always_inline)) -> float {
    if (RAW) return accv;
    float key;
    if (EUC) {
      const float d2 = __builtin_fmaf(-2.0f, accv, kni + qnt[buf * TJ + jl]);
      key = (d2 >= 0.0f) ? -d2 : -INFINITY;
    } else {
      key = accv * a.kscale;
    }
    if (SMP && cdt[buf * TJ + jl] == ti) key = a.mask_key;
    return key;
  };

  // Software-pipelined tile loop: the MFMAs of tile t+1 are issued before the
  // VALU work on tile t, so the matrix and vector pipes overlap within a wave.
  // Tile t lives in LDS buffer t&1; tile t+2 is staged into that buffer once
  // every wave is done with tile t, and tile t+3 is fetched into registers.
  // process(acc, buf, j0) consumes one tile's accumulators; the sweep covers
  // the first ntiles tiles.
  auto sweep = [&](auto&& process, const int ntiles) __attribute__((always_inline)) {
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, PD - 1>;
    f32x16_t accA[NB], accB[NB];
    fetch(0, S0{});
    stash(0, S0{});
    if (ntiles > 1) {
      fetch(1, S1{});
      stash(1, S1{});
    }
    __syncthreads();
    if (ntiles > 2) fetch(2, S0{});
    if (PD == 2 && ntiles > 3) fetch(3, S1{});
    compute(0, accA);
    // step over tile t (t even: buffer / register slot 0, t odd: 1)
    auto step = [&](f32x16_t (&cur)[NB], f32x16_t (&nxt)[NB], int t, auto SLOT)
                    __attribute__((always_inline)) {
      if (t + 1 < ntiles) compute((t + 1) & 1, nxt);
      process(cur, t & 1, t * TJ);
      if (!RAW) __syncthreads();       // process() read this tile's LDS side data
      if (t + 2 < ntiles) {
        stash(t & 1, SLOT);
        if (t + 2 + PD < ntiles) fetch(t + 2 + PD, SLOT);
      }
      __syncthreads();
    };
    for (int t = 0; t < ntiles; t += 2) {
      step(accA, accB, t, S0{});
      if (t + 1 < ntiles) step(accB, accA, t + 1, S1{});
    }
  };

  // Each token's sorted list of packed entries lives in LDS (column `slot`
  // of lst), owned by the lower half-lane: only the drains and the output
  // touch it.  0 marks an empty slot.
  const int slot = wave * 32 + col;
  uint16_t* qidx = reinterpret_cast<uint16_t*>(qent + QC * NT);
  uint64_t* lst = reinterpret_cast<uint64_t*>(qent + QC * NT + QC * NT / 2);
  if (half == 0) {
#pragma unroll
    for (int r = 0; r < KMAX; ++r) lst[r * TPB + slot] = 0;
  }

  if (a.Ksel > 0) {
    // ---------------- pass 1: group-max bound
    float L[KMAX];
    // Short rows (at most 16 tiles): groups of 4 candidates, so that tau is
    // drawn from enough groups to sit close to the K-th key (fewer passers
    // and queue drains in pass 2); long rows: groups of 16.  Long lists on
    // very short rows (K >= 16, at most 8 tiles): every candidate is inserted,
    // tau is the exact K-th key and only about K candidates reach the queues.
    const bool every = KMAX >= 16 && ntiles <= 8;
    const bool fine = ntiles <= 16;
    // Long rows draw the bound from the first three quarters of the tiles (the
    // first quarter for d >= 256 on rows of at least 64 tiles, config 5): any
    // candidates give a valid bound, and the rest of a pass-1 sweep costs more
    // than the extra passers and drains it lets through (c3 select with pass 1
    // over 1/2, 3/4, 7/8, all of the row: 86.1, 83.9, 85.1, 87.6 us; c5 527 -> 490
    // for a quarter against the whole row).
    const int p1 = (NCH * Mfma<T>::KC >= 256 && ntiles >= 64) ? (ntiles + 3) / 4
                                                              : (ntiles > 16 ? (3 * ntiles + 3) / 4 : ntiles);
#pragma unroll
    for (int r = 0; r < KMAX; ++r) L[r] = -INFINITY;
    // MASKED: the tile runs past Nq (only the last one); its extra rows drop out
    auto bound_tile = [&](const f32x16_t (&acc)[NB], int buf, int j0, auto MASKED)
                          __attribute__((always_inline)) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        float key[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int jl = b * 32 + mfma_row(v, lane);
          key[v] = keyof(acc[b][v], buf, jl);
          if (decltype(MASKED)::value && j0 + jl >= a.Nq) key[v] = -INFINITY;
          if (EX && key[v] >= ekey) key[v] = -INFINITY;   // (may drop a tie that is still eligible)
        }
        // keys here are finite or -inf (masked rows, negative euclidean d^2)
        if (every) {
#pragma unroll
          for (int v = 0; v < 16; ++v) bound_insert<KMAX>(L, key[v]);
        } else if (fine) {
#pragma unroll
          for (int g = 0; g < 4; ++g)
            bound_insert<KMAX>(L, max2(max3(key[4 * g], key[4 * g + 1], key[4 * g + 2]), key[4 * g + 3]));
        } else {
          const float m0 = max3(key[0], key[1], key[2]), m1 = max3(key[3], key[4], key[5]);
          const float m2 = max3(key[6], key[7], key[8]), m3 = max3(key[9], key[10], key[11]);
          const float m4 = max3(key[12], key[13], key[14]);
          bound_insert<KMAX>(L, max2(max3(m0, m1, m2), max3(m3, m4, key[15])));
        }
      }
    };
    sweep([&](const f32x16_t (&acc)[NB], int buf, int j0) __attribute__((always_inline)) {
      if (j0 + TJ <= a.Nq)
        bound_tile(acc, buf, j0, std::false_type{});
      else
        bound_tile(acc, buf, j0, std::true_type{});
    }, p1);
    {
      float P[KMAX];
#pragma unroll
      for (int r = 0; r < KMAX; ++r) P[r] = xor32(L[r]);
#pragma unroll
      for (int r = 0; r < KMAX; ++r) bound_insert<KMAX>(L, P[r]);
    }
    float tau = pick<KMAX>(L, a.Ksel - 1);

    // ---------------- pass 2: filter + queue

    uint32_t* myq = qent + tid;
    uint16_t* myqi = qidx + tid;
    // this lane's last written queue slot (one slot before the queue when it
    // is empty), as running LDS pointers: an append is two increments and two
    // stores at the new addresses, no address arithmetic per value
    typedef __attribute__((address_space(3))) uint32_t lds_u32;
    typedef __attribute__((address_space(3))) uint16_t lds_u16;
    lds_u32* const qk0 = (lds_u32*)myq;
    lds_u32* qk = qk0 - NT;
    lds_u16* qi = (lds_u16*)myqi - NT;
    // both half-lanes' queues go into the token's list; only the lower half works
    // Each half-lane inserts its own queue into a list (the lower half starts
    // from the token's stored list, the upper half from an empty one); the
    // lower half then takes the top K of both lists with a bitonic merge:
    // M[r] = max(A[r], B[KP-1-r]) of two descending lists is a bitonic
    // sequence holding the KP largest, which a half-cleaner network sorts.
    auto drain = [&]() __attribute__((always_inline)) {
      const int cnt = (int)((qk - qk0) / NT) + 1;
      float ntau = tau;
      uint64_t L2[KMAX];
#pragma unroll
      for (int r = 0; r < KMAX; ++r) L2[r] = half == 0 ? lst[r * TPB + slot] : 0;
      if constexpr (RAW && !EX && KMAX <= 9) {
        // Raw dot-product keys are finite, so the list can hold float keys
        // (-inf marks an empty slot) kept in order by one med3 per slot, and
        // the indices follow the strict comparisons: a lane's queue holds its
        // candidates in increasing index order and the stored list only earlier
        // candidates, so a later equal key goes after the listed ones, which
        // is the lowest-index-first order.  Packed again for the merge.  (For
        // lists of 16 the packed insertion below measured faster: c5 select
        // 523 against 564 us.)
        float Lk[KMAX];
        uint32_t Li[KMAX];
#pragma unroll
        for (int r = 0; r < KMAX; ++r) {
          Lk[r] = L2[r] == 0 ? -INFINITY : key_of_ord((uint32_t)(L2[r] >> 32));
          Li[r] = ~(uint32_t)L2[r];
        }
        for (int e = 0; __any(e < cnt); ++e) {
          const float xk = (e < cnt) ? __uint_as_float(myq[e * NT]) : -INFINITY;
          const uint32_t xi = myqi[e * NT];
          bool b[KMAX];
#pragma unroll
          for (int r = 0; r < KMAX; ++r) b[r] = xk > Lk[r];
#pragma unroll
          for (int r = KMAX - 1; r >= 1; --r) {
            Lk[r] = __builtin_amdgcn_fmed3f(Lk[r - 1], xk, Lk[r]);
            Li[r] = vsel(b[r], vsel(b[r - 1], Li[r - 1], xi), Li[r]);   // b[r-1] implies b[r]
          }
          Lk[0] = b[0] ? xk : Lk[0];
          Li[0] = vsel(b[0], xi, Li[0]);
        }
#pragma unroll
        for (int r = 0; r < KMAX; ++r) L2[r] = Lk[r] == -INFINITY ? 0 : pack_entry(Lk[r], Li[r]);
      } else {
        for (int e = 0; __any(e < cnt); ++e) {
          const uint64_t x = (e < cnt) ? pack_entry(__uint_as_float(myq[e * NT]), myqi[e * NT]) : 0;
          list_insert<KMAX>(L2, x);
        }
      }
      constexpr int KP = KMAX <= 8 ? 8 : (KMAX <= 16 ? 16 : 32);
      uint64_t M[KP];
#pragma unroll
      for (int r = 0; r < KP; ++r) {
        const int rp = KP - 1 - r;
        uint64_t p = 0;
        if (rp < KMAX) {
          const uint32_t lo = xor32((uint32_t)L2[rp]), hi = xor32((uint32_t)(L2[rp] >> 32));
          p = ((uint64_t)hi << 32) | lo;
        }
        const uint64_t m = r < KMAX ? L2[r] : 0;
        M[r] = m > p ? m : p;
      }
#pragma unroll
      for (int j = KP / 2; j >= 1; j >>= 1)
#pragma unroll
        for (int i = 0; i < KP; ++i)
          if ((i & j) == 0) {
            const uint64_t u = M[i], v = M[i + j];
            M[i] = u > v ? u : v;
            M[i + j] = u > v ? v : u;
          }
      if (half == 0) {
#pragma unroll
        for (int r = 0; r < KMAX; ++r) lst[r * TPB + slot] = M[r];
        const uint64_t kth = pick<KMAX>(reinterpret_cast<const uint64_t(&)[KMAX]>(M), a.Ksel - 1);
        if (kth != 0) ntau = fmaxf(ntau, next_up(key_of_ord((uint32_t)(kth >> 32))));
      }
      tau = from_lower(ntau);
      qk = qk0 - NT;
      qi = (lds_u16*)myqi - NT;
    };
    // Drains are synchronised across the block: a wave that would otherwise
    // drain on its own mid-tile stalls the other waves at the next barrier, so
    // at every tile boundary all waves drain together when any lane of the
    // block holds more than BTHR entries (flags written before the barrier).
    constexpr int BTHR = QC - 6;
    auto filter_tile = [&](const f32x16_t (&acc)[NB], int buf, int j0, auto MASKED)
                           __attribute__((always_inline)) {
      const int t = j0 / TJ;
      if (t > 0) {
        const int* f = dflag + ((t - 1) & 1) * 4;
        if (__any((f[0] | f[1] | f[2] | f[3]) != 0)) drain();
      }
      // candidate index of value v of MFMA block b: jt + b*32 + (v/4)*8 + v%4
      const int jt = j0 + 4 * half;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          if (v % QCHK == 0 && __any(qk >= qk0 + (QC - QCHK) * NT)) drain();
          const int jl = b * 32 + mfma_row(v, lane);
          float key = keyof(acc[b][v], buf, jl);
          if (decltype(MASKED)::value && j0 + jl >= a.Nq) key = __builtin_nanf("");
          // a later round: only candidates ranking after the previous round's last entry
          if (EX && !(key < ekey || (key == ekey && (uint32_t)(j0 + jl) > ej))) key = __builtin_nanf("");
          // (slot <= QC - 1 here: a check precedes every QCHK elements)
          if (PRED_APPEND) {
            // store the passers only; element steps where no lane passes skip it
            if (key >= tau) {
              qk += NT;
              qi += NT;
              // keep the stores on the incremented registers (an add folded
              // into the store offset would leave two live copies to merge)
              asm volatile("" : "+v"(qk), "+v"(qi));
              *qk = __float_as_uint(key);
              *qi = (uint16_t)(jt + (b * 32 + (v >> 2) * 8 + (v & 3)));
            }
          } else {
            // branch-free: write at the current slot, keep it only if it passed
            qk[NT] = __float_as_uint(key);
            qi[NT] = (uint16_t)(jt + (b * 32 + (v >> 2) * 8 + (v & 3)));
            const int adv = (key >= tau) ? NT : 0;
            qk += adv;
            qi += adv;
          }
        }
      }
      const bool need = __any(qk >= qk0 + BTHR * NT);
      if (lane == 0) dflag[(t & 1) * 4 + wave] = need ? 1 : 0;
    };
    sweep([&](const f32x16_t (&acc)[NB], int buf, int j0) __attribute__((always_inline)) {
      if (j0 + TJ <= a.Nq)
        filter_tile(acc, buf, j0, std::false_type{});
      else
        filter_tile(acc, buf, j0, std::true_type{});
    }, ntiles);
    drain();
  }

  // ---------------- the token's list -> idx, vals, w (values kept in registers)
  constexpr int KO = KMAX + OFF;
  float vv[KO], wv[KO];
  int tk[KO];
  int cl[KO];   // sampled: candidate column of each entry (slot 0, the token itself: Nq)
  if (half == 0 && tvalid) {
    if (SMP) {
      tk[0] = ti;
      vv[0] = 1.0f;
      cl[0] = a.Nq;
    }
#pragma unroll
    for (int r = 0; r < KMAX; ++r) {
      const uint64_t ent = lst[r * TPB + slot];
      const float key = key_of_ord((uint32_t)(ent >> 32));
      const int j = (ent == 0 || r >= a.Ksel) ? 0 : (int)(~(uint32_t)ent);
      float val = RAW ? key * a.kscale : key;
      int tok = j;
      if (SMP) tok = a.cand[j];
      if (EUC) val = (key == -INFINITY) ? __builtin_nanf("") : sqrtf(-key);
      if (SMP && EUC && tok == ti) val = a.mask_val;
      vv[OFF + r] = val;
      tk[OFF + r] = tok;
      cl[OFF + r] = j;
    }
    // neighbour weights (layers.py:352-355, 382-385, 394-397, 426-429)
    if (a.softmax) {
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < KO; ++r)
        if (r < a.K) mx = fmaxf(mx, EUC ? -vv[r] : vv[r]);
      float sum = 0.0f;
#pragma unroll
      for (int r = 0; r < KO; ++r) {
        wv[r] = (r < a.K) ? expf((EUC ? -vv[r] : vv[r]) - mx) : 0.0f;
        sum += wv[r];
      }
#pragma unroll
      for (int r = 0; r < KO; ++r) wv[r] = wv[r] / sum;
    } else {
#pragma unroll
      for (int r = 0; r < KO; ++r) wv[r] = EUC ? 1.0f / (vv[r] + 1e-8f) : vv[r];
    }
  }
  // another round follows: hand this round's last entry over in the slot
  // after this round's entries (its first slot)
  const int nxt = OFF + a.kbase + a.Ksel;
  if (nxt < a.K && half == 0 && tvalid) {
    const uint64_t last = lst[(a.Ksel - 1) * TPB + slot];
    const int64_t eo = ((int64_t)bh * a.N + ti) * a.K + nxt;
    a.vals[eo] = __uint_as_float((uint32_t)(last >> 32));
    a.idx[eo] = (int32_t)(uint32_t)last;
  }
  // The block's tokens are consecutive, so each output is one contiguous run
  // of nvalid * K values (one round: the whole rows): staged through LDS (the
  // queue region, free after the final drains) and stored by all threads with
  // consecutive addresses.  This round writes kw entries per token from column
  // c0, register entries rs ...
  uint32_t* stg = qent;
  const int nvalid = min(TPB, a.N - rb * TPB);
  const int rs = a.kbase == 0 ? 0 : OFF;
  const int kw = a.kbase == 0 ? OFF + a.Ksel : a.Ksel;
  const int c0 = a.kbase == 0 ? 0 : OFF + a.kbase;
  const int64_t obase = ((int64_t)bh * a.N + rb * TPB) * a.K;
  auto emit = [&](auto get, uint32_t* dst) __attribute__((always_inline)) {
    __syncthreads();
    if (half == 0 && tvalid) {
#pragma unroll
      for (int r = 0; r < KO; ++r)
        if (r >= rs && r < rs + kw) stg[slot * kw + r - rs] = get(r);
    }
    __syncthreads();
    if (kw == a.K) {
      for (int e = tid; e < nvalid * kw; e += NT) dst[obase + e] = stg[e];
    } else {
      for (int e = tid; e < nvalid * kw; e += NT) {
        const int t = e / kw;
        dst[obase + (int64_t)t * a.K + c0 + (e - t * kw)] = stg[e];
      }
    }
  };
  emit([&](int r) { return (uint32_t)tk[r]; }, reinterpret_cast<uint32_t*>(a.idx));
  emit([&](int r) { return __float_as_uint(vv[r]); }, reinterpret_cast<uint32_t*>(a.vals));
  if (a.w != nullptr) emit([&](int r) { return __float_as_uint(wv[r]); }, reinterpret_cast<uint32_t*>(a.w));
  if (SMP && a.cols != nullptr) emit([&](int r) { return (uint32_t)cl[r]; }, reinterpret_cast<uint32_t*>(a.cols));
}

template <typename T, int NCH, bool EXACT, int KMAX, bool EUC, bool EX = false>
int launch_k(int sampled, const SelArgs& a, hipStream_t s) {
  auto smem = [&](int qc) {
    return 2 * TJ * (a.dkp + SelCfg<T>::VEC) * sizeof(T) + 2 * TJ * (sizeof(float) + sizeof(int)) + 8 * sizeof(int) +
           (size_t)qc * NT * 6 + (size_t)KMAX * TPB * sizeof(uint64_t);
  };
  const dim3 grid(a.BH * a.rb_per_bh);
  if (!sampled)
    hipLaunchKernelGGL((select_kernel<T, NCH, EXACT, KMAX, EUC, false, EX>), grid, dim3(NT),
                       smem(queue_cap<T, NCH, EXACT, KMAX, EUC, false>()), s, a);
  else
    hipLaunchKernelGGL((select_kernel<T, NCH, EXACT, KMAX, EUC, true, EX>), grid, dim3(NT),
                       smem(queue_cap<T, NCH, EXACT, KMAX, EUC, true>()), s, a);
  return (int)hipGetLastError();
}

// Neighbour weights of whole rows after a multi-round selection (the same
// formulas as the single-round kernel: layers.py:352-355, 382-385, 394-397,
// 426-429); one thread per token row.
__global__ __launch_bounds__(256) void sel_weights_kernel(const float* vals, float* w, int64_t rows, int K,
                                                          int softmax, int euclid) {
  const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (row >= rows) return;
  const float* v = vals + row * K;
  float* o = w + row * K;
  if (softmax) {
    float mx = -INFINITY;
    for (int r = 0; r < K; ++r) mx = fmaxf(mx, euclid ? -v[r] : v[r]);
    float sum = 0.0f;
    for (int r = 0; r < K; ++r) sum += expf((euclid ? -v[r] : v[r]) - mx);
    for (int r = 0; r < K; ++r) o[r] = expf((euclid ? -v[r] : v[r]) - mx) / sum;
  } else {
    for (int r = 0; r < K; ++r) o[r] = euclid ? 1.0f / (v[r] + 1e-8f) : v[r];
  }
}

// one list of KMAX entries, or rounds of 32 for wider selections
template <typename T, int NCH, bool EXACT, bool EUC>
int launch_rounds(int sampled, const SelArgs& a, hipStream_t s) {
  if constexpr (EXACT) {
    if (a.Ksel <= 9) return launch_k<T, NCH, EXACT, 9, EUC>(sampled, a, s);
    if (a.Ksel <= 16) return launch_k<T, NCH, EXACT, 16, EUC>(sampled, a, s);
  }
  if (a.Ksel <= 32) return launch_k<T, NCH, EXACT, 32, EUC>(sampled, a, s);
  SelArgs r = a;
  r.w = nullptr;
  for (int base = 0; base < a.Ksel; base += 32) {
    r.kbase = base;
    r.Ksel = min(32, a.Ksel - base);
    const int st = base == 0 ? launch_k<T, NCH, EXACT, 32, EUC, false>(sampled, r, s)
                             : launch_k<T, NCH, EXACT, 32, EUC, true>(sampled, r, s);
    if (st) return st;
  }
  if (a.w != nullptr) {
    const int64_t rows = (int64_t)a.BH * a.N;
    hipLaunchKernelGGL(sel_weights_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, a.vals, a.w,
                       rows, a.K, a.softmax, (int)EUC);
  }
  return (int)hipGetLastError();
}

template <typename T, int NCH, bool EUC>
int launch_n(int sampled, const SelArgs& a, hipStream_t s) {
  return launch_rounds<T, NCH, true, EUC>(sampled, a, s);
}

template <typename T, bool EUC>
int launch_select_t(int sampled, const SelArgs& a, hipStream_t s) {
  if (a.dkp % Mfma<T>::KC != 0 || a.dkp > SelCfg<T>::WIDECH * Mfma<T>::KC || a.dkp % SelCfg<T>::VEC != 0)
    return CNNA_ERR_SHAPE;
  if (a.Nq > 65536) return CNNA_ERR_SHAPE;
  // the queue region also stages one output array (TPB * K <= TPB * 32 values) at the end
  static_assert(TPB * 32 * 2 <= QCMIN * NT * 3, "output staging must fit the queue region");
  const int nch = a.dkp / Mfma<T>::KC;
  constexpr int q = SelCfg<T>::MAXCH / 4;   // head widths 32, 64, 128, 256 (bf16) / 16 .. 128 (f32)
  if (nch == q / 2) return launch_n<T, q / 2, EUC>(sampled, a, s);
  if (nch == q) return launch_n<T, q, EUC>(sampled, a, s);
  if (nch == 2 * q) return launch_n<T, 2 * q, EUC>(sampled, a, s);
  if (nch == 4 * q) return launch_n<T, 4 * q, EUC>(sampled, a, s);
  if constexpr (SelCfg<T>::WIDECH > SelCfg<T>::MAXCH) {
    // float32 heads wider than 128: 256 exactly, or guarded chunks up to 256
    if (nch == SelCfg<T>::WIDECH) return launch_n<T, SelCfg<T>::WIDECH, EUC>(sampled, a, s);
    if (nch > SelCfg<T>::MAXCH) return launch_rounds<T, SelCfg<T>::WIDECH, false, EUC>(sampled, a, s);
  }
  // other widths: guarded chunks, lists of 32
  return launch_rounds<T, SelCfg<T>::MAXCH, false, EUC>(sampled, a, s);
}

}  // namespace
