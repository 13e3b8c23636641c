// Split single-query attention for few streams (gfx950).
//
// One (stream, head) unit of the attention phase keeps one CU busy for the whole visible window:
// at B = 1 the phase of a 16-head model runs on 16 of 256 CUs, reading the head's K and V rows
// (2 L hd floats) through one CU's load pipe.  Here a head runs as S units instead, and the work
// that has to stay sequential -- the sum of the exponentials in key order and each output dim's
// chain of products in key order (SVL/nn/kernels/attention.rs:139-168) -- is the only part that
// is not split:
//   * unit j of head hu scores keys [j Lc, min(L, (j + 1) Lc)), Lc = ceil(L / S), with the
//     16-lane dot of the unsplit unit (thread i of a key's 16 accumulating dims i, i + 16, ...
//     by FMA, then the pairwise lane sum; w_j = scale * dot) and publishes them to the head's row
//     of a score buffer in device memory;
//   * the head's S units meet at a counter in device memory (bounded spin);
//   * each unit forms the softmax of the whole row itself, with the unsplit unit's operations in
//     its order (max; e_j = exp(w_j - max); their sum in key order; e_j / sum), so that every
//     unit of the head holds the same weights, bit for bit;
//   * unit j runs the key-order chains out_d = mul_add(w_k, v_kd, out_d) of dims
//     [j hd / S, (j + 1) hd / S), whose V columns it requested into LDS before the meeting.
// The results equal the unsplit unit's bits.  The units of a launch have to be co-resident; the
// host uses the split only while B * H * S <= the CU count, and a unit whose meeting outlasts the
// spin limit raises the abort flag, writes nothing and ends.
#include "kernels.h"
#include "step_units.h"

namespace svl {

namespace {

constexpr unsigned kMeetSpinLimit = 1u << 22;

// V columns [d0, d0 + DS) of keys 0 .. L - 1 into LDS as [key][DS]: pieces of PB bytes, one per
// lane, rounds of kRowThreads pieces (pieces past the last one repeat it, inside the slack that
// split_v_bytes allocates).
template <int PB>
__device__ __forceinline__ void load_v_columns(const unsigned char* vc, size_t base, int first, int cap, int L,
                                               int row_bytes, int col_bytes, int kbytes, unsigned char* vs) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x % kWave;
  const int ppk = kbytes / PB, np = L * ppk;
  for (int r = 0; r * kRowThreads < np; ++r) {
    const int pc = min(r * kRowThreads + wave * kWave + lane, np - 1);
    const int key = pc / ppk, part = pc % ppk;
    lds_dma<PB, false>(vc + (base + (size_t)((first + key) % cap)) * row_bytes + col_bytes + part * PB,
                       vs + (size_t)(r * kRowThreads + wave * kWave) * PB);
  }
}

template <int HD, bool BF16KV, int S>
__device__ __forceinline__ void attn_split_unit(const AttnArgs& a, int hu, int j, const int* spos, float* scores,
                                                unsigned* abort_flag, unsigned char* smem, RowSync& rs) {
  constexpr int E = BF16KV ? 2 : 4;
  constexpr int C = HD / 16;
  constexpr int DS = HD / S;  // dims of this unit
  static_assert(HD % S == 0 && DS * E >= 4, "split of the head dims");
  const int cap = a.cap, H = a.H, KVH = a.KVH;
  const float scale = a.scale;
  const int h = hu % H, b = hu / H;
  const int li = threadIdx.x % 16, grp = threadIdx.x / 16;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x % kWave;
  float q[C];
  {
    const float* qp = a.q + (size_t)b * H * HD + (size_t)h * HD + li;
#pragma unroll
    for (int c = 0; c < C; ++c) q[c] = ld_co(qp + c * 16);
  }
  const int p = spos[b];
  const int L = visible_keys(a, p);
  const int first = p + 1 - L;
  const size_t kb = a.kv_group > 1 ? (size_t)(b / a.kv_group) : (size_t)b;  // the ring's stream
  const size_t base = (kb * KVH + h / (H / KVH)) * (size_t)cap;             // ring row of slot 0
  float* srow = scores + (size_t)hu * cap;
  // ---- scores of keys [k0, k1): group grp takes keys k0 + grp, k0 + grp + 32, ..., two keys a
  // trip with all their loads in flight together (a key past k1 loads key k1 - 1 and stores
  // nothing, so that every lane of a 16-lane row takes part in the pairwise sum)
  const int Lc = (L + S - 1) / S, k0 = min(L, j * Lc), k1 = min(L, k0 + Lc);
  const unsigned char* kc = (const unsigned char*)a.kc;
  for (int k = k0 + grp; k - grp < k1; k += 64) {
    const int ka = min(k, k1 - 1), kz = min(k + 32, k1 - 1);
    const unsigned char* ra = kc + ((base + (size_t)((first + ka) % cap)) * HD + li) * E;
    const unsigned char* rz = kc + ((base + (size_t)((first + kz) % cap)) * HD + li) * E;
    float xa[C], xz[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if constexpr (BF16KV) {
        xa[c] = bf16_to_f32(ldg((const uint16_t*)ra + 16 * c));
        xz[c] = bf16_to_f32(ldg((const uint16_t*)rz + 16 * c));
      } else {
        xa[c] = ldg((const float*)ra + 16 * c);
        xz[c] = ldg((const float*)rz + 16 * c);
      }
    }
    float acc = 0.0f, acz = 0.0f;
#pragma unroll
    for (int c = 0; c < C; ++c) acc = fmaf(q[c], xa[c], acc);
#pragma unroll
    for (int c = 0; c < C; ++c) acz = fmaf(q[c], xz[c], acz);
    acc = row16_pairwise_sum(acc);
    acz = row16_pairwise_sum(acz);
    if (li == 0 && k < k1) st_co(srow + k, scale * (acc + 0.0f));
    if (li == 0 && k + 32 < k1) st_co(srow + k + 32, scale * (acz + 0.0f));
  }
  __builtin_amdgcn_s_waitcnt(kVmWait0);  // this wave's score stores are complete
  unsigned char* vs = smem;
  constexpr int PB = split_piece_bytes(HD, BF16KV ? 1 : 0, S);
  load_v_columns<PB>((const unsigned char*)a.vc, base, first, cap, L, HD * E, j * DS * E, DS * E, vs);
  float* w = (float*)(smem + split_v_bytes(cap, HD, BF16KV ? 1 : 0, S));
  float* slot = w + cap + kSplitSlack;  // [0, 8): wave maxima; 8: the sum; 9: the meeting's outcome
  // ---- the meeting of the head's units
  rs.sync();  // every row wave's scores are stored
  if (threadIdx.x == 0) {
    unsigned* ctr = a.split_ctr + (size_t)hu * 32;
    __hip_atomic_fetch_add(gbl(ctr), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned spins = 0;
    int ok = 1;
    while ((int)(__hip_atomic_load(gbl(ctr), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - a.split_target) < 0) {
      if (++spins > kMeetSpinLimit) {
        __hip_atomic_store(gbl(abort_flag), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    ((volatile int*)slot)[9] = ok;
  }
  rs.sync();
  if (((volatile int*)slot)[9] == 0) {
    __builtin_amdgcn_s_waitcnt(kVmWait0);  // the direct loads have landed before the wave ends
    return;
  }
  // ---- softmax over the head's L scores, every unit of the head alike
  float mx = -__builtin_huge_valf();
  for (int k = threadIdx.x; k < L; k += kRowThreads) {
    const float v = ld_co(srow + k);
    w[k] = v;
    mx = fmaxf(mx, v);
  }
  mx = wave_max(mx);
  if (lane == 0) slot[wave] = mx;
  rs.sync();
  mx = slot[0];
#pragma unroll
  for (int i = 1; i < kRowWaves; ++i) mx = fmaxf(mx, slot[i]);
  for (int k = threadIdx.x; k < L; k += kRowThreads) w[k] = ref_exp(w[k] - mx);
  rs.sync();
  if (threadIdx.x == 0) slot[8] = ordered_sum_from(w, L, 0.0f);
  rs.sync();
  const float sum = slot[8];
  for (int k = threadIdx.x; k < L; k += kRowThreads) w[k] = w[k] / sum;
  __builtin_amdgcn_s_waitcnt(kVmWait0);  // this wave's V columns have landed
  rs.sync();
  // ---- out_d = mul_add(w_k, v_kd, out_d) over keys in order: lane d of wave 0 owns dim
  // j DS + d; the next 16 keys' operands are read while the current 16 are summed
  if (wave != 0 || lane >= DS) return;
  const float* vf = (const float*)vs + lane;
  const uint16_t* vh = (const uint16_t*)vs + lane;
  auto vload = [&](int k) { return BF16KV ? bf16_to_f32(vh[k * DS]) : vf[k * DS]; };
  // two register sets in turn (keys up to L + 46 < cap + kSplitSlack are read: inside both arrays)
  float wa[16], xa[16], wb[16], xb[16];
  auto read16 = [&](int k, float(&wv)[16], float(&xv)[16]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      wv[i] = w[k + i];
      xv[i] = vload(k + i);
    }
  };
  float acc = 0.0f;
  auto chain16 = [&](int k, const float(&wv)[16], const float(&xv)[16]) {
    if (k + 16 <= L) {
#pragma unroll
      for (int i = 0; i < 16; ++i) acc = fmaf(wv[i], xv[i], acc);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (k + i < L) acc = fmaf(wv[i], xv[i], acc);
    }
  };
  read16(0, wa, xa);
  for (int k = 0; k < L; k += 32) {
    read16(k + 16, wb, xb);
    chain16(k, wa, xa);
    read16(k + 32, wa, xa);
    chain16(k + 16, wb, xb);
  }
  st_co(a.out + (size_t)b * H * HD + (size_t)h * HD + j * DS + lane, acc);
}

}  // namespace

// Launched with the row waves only.  Units u < hheads map to (head hu, part j); with a multiple
// of 8 heads the S units of a head share u % 8, and with it the XCD that dispatch places them on
// (whose L2 then serves the V rows that all of them read).  Units past `hheads` gather the next
// step's audio embedding rows (the first attention phase of an STT step).
template <int AV, int S>
__global__ __launch_bounds__(kRowThreads) void attn_split_kernel(const float* hq, const void* hkc, const void* hvc,
                                                                 const int* hpos, float* hscores, int hcap, int hwindow,
                                                                 int hB, int hheads, const Phase ph, StepParams P,
                                                                 int step) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ WgSync ws;
  init_wg_sync(&ws);
  RowSync rs{&ws, 0u, true};
  const int unit = blockIdx.x;
  if (unit < hheads) {
    constexpr int c = AV - 1;
    const int NH = hheads / S;
    int hu, j;
    if ((NH & 7) == 0) {
      const int r = unit >> 3;
      hu = (unit & 7) + 8 * (r / S);
      j = r % S;
    } else {
      hu = unit / S;
      j = unit % S;
    }
    AttnArgs a = ph.at;
    a.q = hq;
    a.kc = hkc;
    a.vc = hvc;
    a.cap = hcap;
    a.window = hwindow;
    a.B = hB;
    attn_split_unit<(c & 1) ? 128 : 64, (c & 2) != 0, S>(a, hu, j, hpos, hscores, &P.sync->abort_flag[0], smem, rs);
  } else if (step + 1 < P.n_steps && !P.text) {
    gather_unit(ph.e, P.audio + (size_t)(step + 1) * P.audio_stride, unit - hheads);
  }
}

using SplitKernel = void (*)(const float*, const void*, const void*, const int*, float*, int, int, int, int, const Phase,
                             StepParams, int);

template <int S>
SplitKernel split_kernel_for(int av) {
  switch (av) {
    case 1: return attn_split_kernel<1, S>;
    case 2: return attn_split_kernel<2, S>;
    case 3: return attn_split_kernel<3, S>;
    default: return attn_split_kernel<4, S>;
  }
}

hipError_t launch_attn_split(const Phase& ph, const StepParams& p, int step, int S, float* scores, hipStream_t s) {
  const AttnArgs& a = ph.at;
  const int hd = a.hd == 128 ? 128 : 64;
  if (a.hd != hd || !a.split_ctr || !scores) return hipErrorInvalidValue;
  const int av = attn_variant(hd, a.kv_bf16, 1);
  SplitKernel k;
  switch (S) {
    case 2: k = split_kernel_for<2>(av); break;
    case 4: k = split_kernel_for<4>(av); break;
    case 8: k = split_kernel_for<8>(av); break;
    case 16: k = split_kernel_for<16>(av); break;
    default: return hipErrorInvalidValue;
  }
  const int nh = a.B * a.H, gather = ph.units - nh / a.hpu;
  hipLaunchKernelGGL(k, dim3(nh * S + gather), dim3(kRowThreads), split_smem(a.cap, hd, a.kv_bf16, S), s, a.q, a.kc,
                     a.vc, (const int*)p.pos, scores, a.cap, a.window, a.B, nh * S, ph, p, step);
  return hipGetLastError();
}

}  // namespace svl
