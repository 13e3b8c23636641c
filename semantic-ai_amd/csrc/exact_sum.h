// Element-order row sums, as candle-nn's CPU RmsNorm / LayerNorm compute their statistics: one
// f32 accumulator, x_0, x_1, ... added in index order.  With quantized activations the greedy
// tokens depend on the last bit of these sums, so the kernels reproduce the sequential rounding
// exactly -- but a plain dependent chain costs ~6 cycles per element (2048 elements: 5 us).
//
// Sum of squares (non-negative terms), exactly and mostly in parallel.  While the running sum
// S stays in one binade [2^E, 2^(E+1)), every partial sum is a multiple of u = 2^(E-23) and
// fl(S + t) = S + rint(t / u) u (ties aside: they round to the even multiple, which depends on
// S).  So a chunk of terms whose partial sums stay in one binade adds the integer
// A = sum rint(t_i / u) -- computable from the chunk alone once E is known -- and chunks combine
// by an exact (f64) prefix sum.  The row is cut into chunks of 8; each chunk's binade is taken
// from an approximate prefix sum, and a chunk is "special" when that guess is unsafe: the first
// chunk, a start below 2^-100, a start or end within 2^-9 (relative) of a binade edge, or a
// tie.  Special chunks (about 14 of 256 for a row of 2048 normal values) are added sequentially
// in f32 from their exact start, in chunk order; every other chunk is then verified against its
// exact start (start in binade E, start + A u below 2^(E+1), which bounds every partial sum
// since the terms are >= 0).  Any failed check -- a guess that did not hold, an f64 sum that
// could round, a non-finite or huge term -- falls back to the plain sequential chain, so the
// result is the sequential sum in every case.
#pragma once

#include "device_math.h"

namespace svl {

constexpr int kSumChunk = 8;

// Lane-segment layout of a staged row: element i of a row of K at i + 4 (i / (8 Q)), so that lane
// j of the summing wave owns elements [8 Q j, 8 Q (j + 1)) (Q chunks of 8) contiguously, and the
// 16-byte reads of consecutive lanes fall on distinct LDS banks.  Q is chosen per call site
// with 512 Q >= K (K <= 64 lanes x 8 Q).
template <int Q>
__device__ __forceinline__ int seg_pos(int i) {
  return i + 4 * (i / (kSumChunk * Q));
}

// LDS floats of one staged array: the padded row (it also covers the reads of the last, partial
// segment), or the summing wave's list of special chunks (at most 64 entries of 48 bytes).
__host__ __device__ constexpr int staged_floats(int K) { return K + 768; }

typedef float sum_v4 __attribute__((ext_vector_type(4)));

// acc += t[i] for i = 0 .. n - 1 in order (t 16-byte aligned, LDS), reading 16 values ahead.
__device__ __forceinline__ float ordered_sum_from(const float* t, int n, float acc) {
  const sum_v4* t4 = (const sum_v4*)t;
  const int n16 = n / 16;
  sum_v4 cur[4], nxt[4];
  if (n16 > 0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) cur[u] = t4[u];
  }
  for (int c = 0; c < n16; ++c) {
    if (c + 1 < n16) {
#pragma unroll
      for (int u = 0; u < 4; ++u) nxt[u] = t4[(c + 1) * 4 + u];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc = acc + cur[u].x;
      acc = acc + cur[u].y;
      acc = acc + cur[u].z;
      acc = acc + cur[u].w;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) cur[u] = nxt[u];
  }
  for (int i = n16 * 16; i < n; ++i) acc = acc + t[i];
  return acc;
}

// The plain sequential sum of a staged row (every lane runs it on its own `arr`).
template <int Q>
__device__ __forceinline__ float staged_sequential_sum(const float* arr, int K) {
  constexpr int SEG = kSumChunk * Q;
  float acc = 0.0f;
  for (int s = 0; s * SEG < K; ++s) acc = ordered_sum_from(arr + s * (SEG + 4), min(SEG, K - s * SEG), acc);
  return acc;
}

__device__ __forceinline__ int exp_of(float x) {  // floor(log2 x) for normal x > 0
  return __builtin_amdgcn_frexp_expf(x) - 1;
}

// Inclusive scans over the 64 lanes of a wave with DPP (row_shr 1, 2, 4, 8 within rows of 16,
// then row_bcast 15 and 31 across rows): six VALU steps, no LDS round trip.  `old` 0 and
// bound_ctrl make disabled or out-of-row sources contribute the identity (0 for sums).
template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp0(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWS, 0xf, true);
}

template <int CTRL, int ROWS>
__device__ __forceinline__ double dpp0(double v) {
  const long long b = __builtin_bit_cast(long long, v);
  const int lo = dpp0<CTRL, ROWS>((int)b), hi = dpp0<CTRL, ROWS>((int)(b >> 32));
  return __builtin_bit_cast(double, (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}

template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp0(float v) {
  return __int_as_float(dpp0<CTRL, ROWS>(__float_as_int(v)));
}

template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v) {
  v = v + dpp0<0x111, 0xf>(v);  // row_shr:1
  v = v + dpp0<0x112, 0xf>(v);  // row_shr:2
  v = v + dpp0<0x114, 0xf>(v);  // row_shr:4
  v = v + dpp0<0x118, 0xf>(v);  // row_shr:8
  v = v + dpp0<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v = v + dpp0<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const long long b = __builtin_bit_cast(long long, v);
  const int lo = __builtin_amdgcn_readlane((int)b, lane), hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
  return __builtin_bit_cast(double, (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}

__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Wave minimum / maximum of an int (lane 63 of a DPP scan holds it; broadcast from there).
__device__ __forceinline__ int wave_min(int v) {
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x111, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x112, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x114, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x118, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x142, 0xa, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x143, 0xc, 0xf, false));
  return __builtin_amdgcn_readlane(v, kWave - 1);
}

__device__ __forceinline__ int wave_max(int v) { return -wave_min(-v); }

// Sequential f32 sum of the staged squares `sq` (K >= 1 terms, Q chunks of 8 per lane) by one
// full wave; every lane returns the same value.  `scratch` is LDS for the list of special chunks
// (48 bytes each, at most 64 of them; 16-byte aligned).
template <int Q>
__device__ __forceinline__ float exact_sum_squares(const float* sq, int K, unsigned char* scratch) {
  constexpr int SEG = kSumChunk * Q;
  const int lane = threadIdx.x & (kWave - 1);
  const int G = (K + kSumChunk - 1) / kSumChunk;
  // this lane's chunks g = Q lane + q, elements 8 g .. 8 g + 7 (0 past K)
  float t[Q][kSumChunk];
  const float* seg = sq + lane * (SEG + 4);
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int i0 = lane * SEG + q * kSumChunk;
    sum_v4 a = {0.0f, 0.0f, 0.0f, 0.0f}, b = a;
    if (i0 < K) {
      a = *(const sum_v4*)(seg + q * kSumChunk);
      b = *(const sum_v4*)(seg + q * kSumChunk + 4);
    }
    t[q][0] = a.x; t[q][1] = a.y; t[q][2] = a.z; t[q][3] = a.w;
    t[q][4] = b.x; t[q][5] = b.y; t[q][6] = b.z; t[q][7] = b.w;
#pragma unroll
    for (int e = 0; e < kSumChunk; ++e)
      if (i0 + e >= K) t[q][e] = 0.0f;
  }
  // approximate chunk sums and starts (any order: they only pick the binade)
  bool bad = false;
  float c[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    float s4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) s4[e] = t[q][e] + t[q][e + 4];
    c[q] = (s4[0] + s4[2]) + (s4[1] + s4[3]);
#pragma unroll
    for (int e = 0; e < kSumChunk; ++e) bad |= !(t[q][e] <= 0x1p100f);  // non-finite or huge
  }
  float lt = 0.0f;
#pragma unroll
  for (int q = 0; q < Q; ++q) lt = lt + c[q];
  float run = wave_incl_scan(lt) - lt;  // approximate exclusive prefix
  // classification, and for ordinary chunks the exact increment D = A u
  unsigned spmask = 0;  // bit q: chunk q of this lane is special
  double D[Q];
  int E[Q];
  int emin = 1 << 20, emax = -(1 << 20);
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int g = lane * Q + q;
    const float P = run;
    run = run + c[q];
    D[q] = 0.0;
    E[q] = 0;
    if (g >= G) continue;  // empty chunk past the row
    bool sp = g == 0 || !(P >= 0x1p-100f);
    const int e = exp_of(P);
    const float lo = __builtin_ldexpf(1.0f, e), hi = __builtin_ldexpf(1.0f, e + 1);
    sp |= P < lo * (1.0f + 0x1p-9f) || P + c[q] > hi * (1.0f - 0x1p-9f);
    float A0 = 0.0f, A1 = 0.0f;
    bool tie = false;
#pragma unroll
    for (int k = 0; k < kSumChunk; ++k) {
      const float y = __builtin_ldexpf(t[q][k], 23 - e);
      const float r = __builtin_rintf(y);
      if (k & 1) A1 = A1 + r;
      else A0 = A0 + r;
      tie |= fabsf(y - r) == 0.5f;
    }
    sp |= tie;
    if (sp) {
      spmask |= 1u << q;
    } else {
      E[q] = e;
      D[q] = __builtin_ldexp((double)(A0 + A1), e - 23);  // integers below 2^24: the f32 sum is exact
      emin = min(emin, e);
      emax = max(emax, e);
    }
  }
  // wave-uniform guards: huge terms, or binades too far apart for exact f64 sums
  emin = wave_min(emin);
  emax = wave_max(emax);
  if (__any(bad) || (emax >= emin && emax - emin > 28)) return staged_sequential_sum<Q>(sq, K);
  // exact exclusive prefix of D over chunks (specials contribute 0 here)
  double ld = 0.0;
#pragma unroll
  for (int q = 0; q < Q; ++q) ld = ld + D[q];
  const double lincl = wave_incl_scan(ld);
  const double total_d = readlane_f64(lincl, kWave - 1);
  double sp_run = lincl - ld;  // exact: the same multiples of 2^(emin-23)
  double Sp[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    Sp[q] = sp_run;
    sp_run = sp_run + D[q];
  }
  // the specials in chunk order (lane-major, g = Q lane + q): each owning lane writes its terms
  // and Sp at the special's rank in an LDS list
  const int cnt = __builtin_popcount(spmask);
  const int cincl = wave_incl_scan(cnt);
  const int nspecial = __builtin_amdgcn_readlane(cincl, kWave - 1);
  const int before0 = cincl - cnt;  // specials before this lane's first chunk
  if (nspecial > kWave) return staged_sequential_sum<Q>(sq, K);  // rows built to defeat the guesses
  struct Entry {
    sum_v4 a, b;
    double sp;
    float gap, pad;
  };
  Entry* list = (Entry*)scratch;  // [nspecial rounded up to 8], 48 bytes each
  const int nlist = (nspecial + 7) & ~7;
  {
    int r = before0;
#pragma unroll
    for (int q = 0; q < Q; ++q)
      if (spmask & (1u << q)) {
        list[r].a = sum_v4{t[q][0], t[q][1], t[q][2], t[q][3]};
        list[r].b = sum_v4{t[q][4], t[q][5], t[q][6], t[q][7]};
        list[r].sp = Sp[q];
        ++r;
      }
    // zero entries up to a multiple of 8: they add +0 to a non-negative sum, which changes nothing
    if (lane >= nspecial && lane < nlist) {
      list[lane].a = sum_v4{0.0f, 0.0f, 0.0f, 0.0f};
      list[lane].b = list[lane].a;
      list[lane].sp = 0.0;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  // A special's start is the previous special's end plus the ordinary chunks between them,
  // end_{k-1} + gap_k, gap_k = Sp_k - Sp_{k-1}.  Those chunks all lie in one binade E (an edge
  // would have made one of them special), so gap_k is a multiple of 2^(E-23) below 2^(E+1) --
  // an f32 -- and end_{k-1} + gap_k is an exact f32 add.  Lane k prepares gap_k; the serial pass
  // is then nine dependent f32 adds per special, and lane k checks afterwards, in parallel, that
  // its gap and its start were exact.
  double my_sp = 0.0;
  float my_gap = 0.0f;
  bool inexact = false;
  if (lane < nspecial) my_sp = list[lane].sp;
  {
    const double sp_prev = __shfl_up(my_sp, 1, kWave);
    const double gap = lane == 0 ? my_sp : my_sp - sp_prev;  // exact: multiples of 2^(emin-23)
    my_gap = (float)gap;
    if (lane < nspecial) inexact = (double)my_gap != gap;
    if (lane < nlist) list[lane].gap = lane < nspecial ? my_gap : 0.0f;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  // serial pass (uniform across the wave); terms past K and padding entries are 0 and add nothing
  float end = 0.0f, my_end_f = 0.0f;
  constexpr int kBatch = 8;  // entries loaded together, before the batch's additions
  for (int k0 = 0; k0 < nlist; k0 += kBatch) {
    sum_v4 a[kBatch], b[kBatch];
    float gp[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      a[i] = list[k0 + i].a;
      b[i] = list[k0 + i].b;
      gp[i] = list[k0 + i].gap;
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      float s = end + gp[i];
      s = s + a[i].x;
      s = s + a[i].y;
      s = s + a[i].z;
      s = s + a[i].w;
      s = s + b[i].x;
      s = s + b[i].y;
      s = s + b[i].z;
      s = s + b[i].w;
      my_end_f = lane == k0 + i ? s : my_end_f;
      end = s;
    }
  }
  // lane k: was end_{k-1} + gap_k exact?  The f64 sum is exact when end_{k-1}'s lowest bit is
  // >= 2^(emax-51) (the gap is nonzero only right after an ordinary chunk, below 2^(emax+1)).
  const double my_end = (double)my_end_f;
  {
    const float e_prev = __shfl_up(my_end_f, 1, kWave);
    const float pe = lane == 0 ? 0.0f : e_prev;
    const float start = pe + my_gap;
    if (lane < nspecial) {
      if (my_gap != 0.0f && pe != 0.0f && !(pe >= 0x1p-126f && exp_of(pe) >= emax - 28)) inexact = true;
      inexact |= (double)start != (double)pe + (double)my_gap;
    }
  }
  inexact = __any(inexact);
  // verify every ordinary chunk against its exact start: the last special's end plus the
  // ordinary chunks since (chunk 0 is always special, so an ordinary chunk has before >= 1).
  // The shuffles run on every lane (a lane-exchange from an inactive lane reads 0).
  bool fail = inexact;
  int before = before0;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int src = max(before - 1, 0);
    const double e_k = __shfl(my_end, src, kWave), sp_k = __shfl(my_sp, src, kWave);
    const bool spq = (spmask >> q) & 1u;
    if (!spq && lane * Q + q < G) {
      // exact whenever the start can pass (e_k below 2^(E+1))
      const double st = e_k + (Sp[q] - sp_k);
      const double lo = __builtin_ldexp(1.0, E[q]), hi = __builtin_ldexp(1.0, E[q] + 1);
      fail |= !(st >= lo && st < hi && st + D[q] < hi);
    }
    before += spq ? 1 : 0;
  }
  if (__any(fail)) return staged_sequential_sum<Q>(sq, K);
  const double S = readlane_f64(my_end, nspecial - 1) + (total_d - readlane_f64(my_sp, nspecial - 1));
  const float out = (float)S;
  if ((double)out != S) return staged_sequential_sum<Q>(sq, K);
  return out;
}

}  // namespace svl
