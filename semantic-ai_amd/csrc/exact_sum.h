// Element-order row sums, as candle-nn's CPU RmsNorm / LayerNorm compute their statistics: one
// f32 accumulator, x_0, x_1, ... added in index order.  With quantized activations the greedy
// tokens depend on the last bit of these sums, so the kernels reproduce the sequential rounding
// exactly -- but a plain dependent chain costs ~6 cycles per element (2048 elements: 5 us, 11 us
// when fed from LDS).
//
// Sum of squares (non-negative terms), exactly and mostly in parallel, by the 8 row waves of a
// workgroup.  While the running sum S stays in one binade [2^E, 2^(E+1)), every partial sum is a
// multiple of u = 2^(E-23) and fl(S + t) = S + rint(t / u) u (ties aside: they round to the even
// multiple, which depends on S).  So a chunk of terms whose partial sums stay in one binade adds
// the integer A = sum rint(t_i / u) -- computable from the chunk alone once E is known -- and
// chunks combine by an exact (f64) prefix sum.  The row is cut into chunks of 4 (one per thread
// and slab of 2048 elements); each chunk's binade is taken from an approximate prefix sum, and a
// chunk is "special" when that guess is unsafe: the first chunk, a start below 2^-120, a start or
// end within 2^-9 (relative) of a binade edge, or a tie.  A chunk of zeros adds exactly 0 and is
// never special.  Special chunks (about 17 of 512 for a row of 2048 normal values) are added
// sequentially in f32 by one wave from their exact start, in chunk order; every other chunk is
// then verified against its exact start (start in binade E, start + A u below 2^(E+1), which
// bounds every partial sum since the terms are >= 0).  Any failed check -- a guess that did not
// hold, an f64 sum that could round, a non-finite or huge term, too many specials -- falls back
// to the plain sequential chain, so the result is the sequential sum in every case.
#pragma once

#include "device_math.h"

namespace svl {

typedef float sum_v4 __attribute__((ext_vector_type(4)));

// LDS floats of one staged array of a row of K: the row itself (contiguous, 16-byte aligned), or
// the summing workgroup's scratch (block-scan partials and the list of special chunks).
__host__ __device__ constexpr int staged_floats(int K) { return K + 768; }

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

// Wave minimum of an int (lane 63 of a DPP scan holds it; broadcast from there).
__device__ __forceinline__ int wave_min(int v) {
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x111, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x112, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x114, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x118, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x142, 0xa, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x143, 0xc, 0xf, false));
  return __builtin_amdgcn_readlane(v, kWave - 1);
}

// The LDS the block sum works in (`scratch`, staged_floats(K) floats): per-wave partials, then the
// list of special chunks.
struct SumPartials {
  float approx[4][8];  // approximate chunk-sum totals per slab and wave
  double exact[4][8];  // exact increment totals per slab and wave
  int count[4][8];     // special chunks per slab and wave
  int bad[4][8];       // non-finite or huge terms per slab and wave
  int fail;
  float result;
};

struct SumEntry {  // one special chunk: its terms, Sp (the ordinary increments before it),
  sum_v4 t;        // and, after the serial pass, the exact sum at its end
  double sp;
  float end;
  float pad;
};

constexpr int kSumWaves = 8;
constexpr int kSumThreads = kSumWaves * kWave;  // the 512 row threads
constexpr int kSlab = 4 * kSumThreads;          // elements per slab: one chunk of 4 per thread
constexpr int kSumPartialsBytes = (int)((sizeof(SumPartials) + 15) & ~(size_t)15);

// Special chunks the list holds for a row of K (the serial pass has to stay short anyway).
__host__ __device__ constexpr int sum_list_capacity(int K) {
  return (staged_floats(K) * 4 - kSumPartialsBytes) / (int)sizeof(SumEntry) < 256
             ? (staged_floats(K) * 4 - kSumPartialsBytes) / (int)sizeof(SumEntry)
             : 256;
}

__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ double shfl_up1_f64(double v) {  // lane l gets lane l - 1's value (lane 0: its own)
  const long long b = __builtin_bit_cast(long long, v);
  const int src = (int)((threadIdx.x & (kWave - 1)) == 0 ? threadIdx.x & (kWave - 1) : (threadIdx.x & (kWave - 1)) - 1) * 4;
  const int lo = __builtin_amdgcn_ds_bpermute(src, (int)b), hi = __builtin_amdgcn_ds_bpermute(src, (int)(b >> 32));
  return __builtin_bit_cast(double, (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}

__device__ __forceinline__ float shfl_up1_f32(float v) {
  const int l = threadIdx.x & (kWave - 1);
  return __int_as_float(__builtin_amdgcn_ds_bpermute((l == 0 ? 0 : l - 1) * 4, __float_as_int(v)));
}

// Sequential f32 sum of the staged squares sq[0, K) (contiguous, 16-byte aligned, K % 4 == 0,
// K <= 2048 U) by the kSumThreads row threads, which all call it and all get the result.
// `sync` is the row threads' barrier.  `scratch` is LDS of staged_floats(K) floats.
//
// Binade guards without reductions: every ordinary chunk's binade E lies in [Ea - 26, Ea + 1],
// Ea = the binade of the approximate row total (known to every thread after the first barrier),
// so the increments are multiples of 2^(Ea-49); with their total below 2^(Ea+3) (checked), every
// partial sum of them, in any order, is exact in f64.
template <int U, class Sync>
__device__ __forceinline__ float block_exact_sum_squares(const float* sq, int K, unsigned char* scratch, Sync& sync) {
  static_assert(U >= 1 && U <= 4, "rows of at most 8192 elements");
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int NC = K / 4;  // chunks
  SumPartials* part = (SumPartials*)scratch;
  SumEntry* list = (SumEntry*)(scratch + kSumPartialsBytes);
  const int cap = sum_list_capacity(K);
  // ---- this thread's chunks c = tid + 512 u (slab u), elements 4 c .. 4 c + 3
  sum_v4 t[U];
  float c4[U];
  bool bad = false;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int c = tid + kSumThreads * u;
    t[u] = c < NC ? ((const sum_v4*)sq)[c] : sum_v4{0.0f, 0.0f, 0.0f, 0.0f};
    c4[u] = (t[u].x + t[u].y) + (t[u].z + t[u].w);
    bad |= !(t[u].x <= 0x1p120f) | !(t[u].y <= 0x1p120f) | !(t[u].z <= 0x1p120f) | !(t[u].w <= 0x1p120f);
  }
  // ---- approximate exclusive prefix of the chunk sums (any order: it only picks the binade)
  float wincl[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    wincl[u] = wave_incl_scan(c4[u]);
    if (lane == kWave - 1) part->approx[u][wave] = wincl[u];
  }
  if (tid == 0) part->fail = 0;
  sync.sync();
  float P[U];
  float ptotal = 0.0f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float wave_off = 0.0f, slab_total = 0.0f;
#pragma unroll
    for (int w = 0; w < kSumWaves; ++w) {
      const float v = part->approx[u][w];
      if (w < wave) wave_off = wave_off + v;
      slab_total = slab_total + v;
    }
    P[u] = ptotal + wave_off + (wincl[u] - c4[u]);
    ptotal = ptotal + slab_total;
  }
  const int ea = ptotal >= 0x1p-120f ? exp_of(ptotal) : -1000;
  // ---- classification; an ordinary chunk's exact increment D = A 2^(E-23)
  bool sp[U], live[U];
  double D[U];
  int E[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int c = tid + kSumThreads * u;
    sp[u] = false;
    live[u] = false;  // a chunk past the row or of zeros adds exactly 0 wherever it starts
    D[u] = 0.0;
    E[u] = 0;
    if (c >= NC || (c > 0 && c4[u] == 0.0f)) continue;
    live[u] = true;
    const int e = exp_of(P[u]);
    bool s = c == 0 || !(P[u] >= 0x1p-120f) || e < ea - 26 || e > ea + 1;
    const float lo = __builtin_ldexpf(1.0f, e), hi = __builtin_ldexpf(1.0f, e + 1);
    s |= P[u] < lo * (1.0f + 0x1p-9f) || P[u] + c4[u] > hi * (1.0f - 0x1p-9f);
    const float y0 = __builtin_ldexpf(t[u].x, 23 - e), y1 = __builtin_ldexpf(t[u].y, 23 - e);
    const float y2 = __builtin_ldexpf(t[u].z, 23 - e), y3 = __builtin_ldexpf(t[u].w, 23 - e);
    const float r0 = __builtin_rintf(y0), r1 = __builtin_rintf(y1), r2 = __builtin_rintf(y2), r3 = __builtin_rintf(y3);
    s |= fabsf(y0 - r0) == 0.5f || fabsf(y1 - r1) == 0.5f || fabsf(y2 - r2) == 0.5f || fabsf(y3 - r3) == 0.5f;
    sp[u] = s;
    if (!s) {
      E[u] = e;
      D[u] = __builtin_ldexp((double)((r0 + r1) + (r2 + r3)), e - 23);  // integers below 2^24: exact
    }
  }
  // ---- exact prefix of D within the wave; specials ranked by ballot
  double dincl[U];
  int wrank[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    dincl[u] = wave_incl_scan(D[u]);
    const unsigned long long m = __ballot(sp[u]);
    wrank[u] = __builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u));
    if (lane == kWave - 1) part->exact[u][wave] = dincl[u];
    if (lane == 0) part->count[u][wave] = __popcll(m);
  }
  {
    const unsigned long long mb = __ballot(bad);
    if (lane == 0) part->bad[0][wave] = mb != 0ull;
  }
  sync.sync();
  // ---- global exact prefix Sp, rank, totals (every thread reads the same partials)
  double Sp[U];
  int rank[U];
  double total_d = 0.0;
  int nspecial = 0;
  bool anybad = false;
#pragma unroll
  for (int w = 0; w < kSumWaves; ++w) anybad |= part->bad[0][w] != 0;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    double doff = 0.0, dslab = 0.0;
    int coff = 0, cslab = 0;
#pragma unroll
    for (int w = 0; w < kSumWaves; ++w) {
      const double dv = part->exact[u][w];
      const int cv = part->count[u][w];
      if (w < wave) {
        doff = doff + dv;
        coff += cv;
      }
      dslab = dslab + dv;
      cslab += cv;
    }
    Sp[u] = total_d + doff + (dincl[u] - D[u]);
    rank[u] = nspecial + coff + wrank[u];
    total_d = total_d + dslab;
    nspecial += cslab;
  }
  const bool ok = !anybad && (K & 3) == 0 && K <= kSlab * U && nspecial >= 1 && nspecial <= cap &&
                  total_d < __builtin_ldexp(1.0, ea + 3);
  if (ok) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (sp[u]) {
        list[rank[u]].t = t[u];
        list[rank[u]].sp = Sp[u];
      }
  }
  sync.sync();
  bool fail = !ok;
  if (ok && wave == 0) {
    // ---- serial pass: a special's start is the previous special's end plus the ordinary chunks
    // between them, end_{k-1} + gap_k, gap_k = Sp_k - Sp_{k-1}.  Those chunks lie in one binade
    // (an edge would have made one of them special), so gap_k is a multiple of its ulp below
    // 2^(E+1) -- an f32 -- and end_{k-1} + gap_k is an exact f32 add (checked below).  Lane j
    // holds special base + j; the chain reads the operands with readlane (lanes past the list
    // hold zeros: adding +0 leaves the sum unchanged).
    float end = 0.0f;
    double carry_sp = 0.0;
    float carry_end = 0.0f;
    for (int base = 0; base < nspecial; base += kWave) {
      const int j = base + lane;
      const bool in = j < nspecial;
      const sum_v4 tv = in ? list[j].t : sum_v4{0.0f, 0.0f, 0.0f, 0.0f};
      const double spj = list[in ? j : nspecial - 1].sp;  // past the list: gap 0
      double spp = shfl_up1_f64(spj);
      if (lane == 0) spp = carry_sp;
      const double gap = spj - spp;
      const float gapf = (float)gap;
      float my_end = 0.0f;
      const int n_here = min(kWave, nspecial - base);
      for (int k = 0; k < n_here; k += 8) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float s = end + readlane_f32(gapf, k + i);
          s = s + readlane_f32(tv.x, k + i);
          s = s + readlane_f32(tv.y, k + i);
          s = s + readlane_f32(tv.z, k + i);
          s = s + readlane_f32(tv.w, k + i);
          my_end = lane == k + i ? s : my_end;
          end = s;
        }
      }
      // each special's start was an exact f32 add (the f64 sum is exact when the previous end's
      // lowest bit is >= 2^(Ea-49); the gap is nonzero only right after an ordinary chunk)
      float pe = shfl_up1_f32(my_end);
      if (lane == 0) pe = carry_end;
      if (in) {
        if (gap != 0.0 && pe != 0.0f && !(pe >= 0x1p-126f && exp_of(pe) >= ea - 26)) fail = true;
        fail |= (double)gapf != gap || (double)(pe + gapf) != (double)pe + gap;
        list[j].end = my_end;
      }
      carry_sp = readlane_f64(spj, kWave - 1);
      carry_end = readlane_f32(my_end, kWave - 1);
    }
  }
  sync.sync();
  if (ok) {
    // ---- every ordinary chunk against its exact start: the last special's end plus the
    // ordinary chunks since (chunk 0 is always special, so rank >= 1); exact whenever it can pass
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (sp[u] || !live[u]) continue;
      const SumEntry& last = list[rank[u] - 1];
      const double st = (double)last.end + (Sp[u] - last.sp);
      const double lo = __builtin_ldexp(1.0, E[u]), hi = __builtin_ldexp(1.0, E[u] + 1);
      fail |= !(st >= lo && st < hi && st + D[u] < hi);
    }
    if (__any(fail) && lane == 0) part->fail = 1;
  }
  sync.sync();
  if (ok && !part->fail) {
    const SumEntry& last = list[nspecial - 1];
    const double S = (double)last.end + (total_d - last.sp);
    const float out = (float)S;
    if ((double)out == S) return out;  // uniform: every thread computed the same S
  }
  // ---- fallback: the plain sequential chain by wave 0, published through the scratch
  if (wave == 0) {
    const float acc = ordered_sum_from(sq, K, 0.0f);
    if (lane == 0) part->result = acc;
  }
  sync.sync_long();
  return part->result;
}

}  // namespace svl
