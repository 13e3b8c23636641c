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
//     by FMA, then the pairwise lane sum; w_j = scale * dot) and publishes each score with the
//     launch's tag in the head's row of a score buffer in device memory (one 8-byte store);
//   * every unit reads the whole row back, reading an entry again until it carries the launch's
//     tag (bounded), so that no counter round trip separates publishing from reading;
//   * each unit forms the softmax of the whole row itself, with the unsplit unit's operations in
//     its order (max; e_j = exp(w_j - max); their sum in key order; e_j / sum), so that every
//     unit of the head holds the same weights, bit for bit;
//   * unit j runs the key-order chains out_d = mul_add(w_k, v_kd, out_d) of dims
//     [j hd / S, (j + 1) hd / S), whose V columns it requested into LDS, one row of keys per
//     dim, before reading the scores.
// The results equal the unsplit unit's bits.  The units of a head have to be co-resident; the
// host uses the split only while B * H * S <= the CU count, and a unit whose wait for the scores
// outlasts the spin limit raises the abort flag, writes nothing and ends.
#include "kernels.h"
#include "step_units.h"

namespace svl {

namespace {

// acc + t[0] + t[1] + ... + t[n - 1], in that order (t in LDS, 16-byte aligned, with 16 readable
// floats past n).  The 16-value batches run as a loop in assembly: a batch's four 16-byte reads
// are issued while the batch before it is summed (register sets v64-v79 and v80-v95 in turn), so
// that the sum advances at close to the rate of its dependent adds; the last n % 16 values follow
// in C++.
__device__ __forceinline__ float ordered_sum_lds(const float* t, int n, float acc) {
  int n16 = __builtin_amdgcn_readfirstlane(n >> 4);
  uint32_t ta = lds_addr(t);
  if (n16 > 0) {
    asm volatile(
        "ds_read_b128 v[64:67], %[t]\n\t"
        "ds_read_b128 v[68:71], %[t] offset:16\n\t"
        "ds_read_b128 v[72:75], %[t] offset:32\n\t"
        "ds_read_b128 v[76:79], %[t] offset:48\n\t"
        "1:\n\t"
        "s_waitcnt lgkmcnt(0)\n\t"
        "ds_read_b128 v[80:83], %[t] offset:64\n\t"
        "v_add_f32 %[acc], %[acc], v64\n\t"
        "ds_read_b128 v[84:87], %[t] offset:80\n\t"
        "v_add_f32 %[acc], %[acc], v65\n\t"
        "ds_read_b128 v[88:91], %[t] offset:96\n\t"
        "v_add_f32 %[acc], %[acc], v66\n\t"
        "ds_read_b128 v[92:95], %[t] offset:112\n\t"
        "v_add_f32 %[acc], %[acc], v67\n\t"
        "v_add_f32 %[acc], %[acc], v68\n\t"
        "v_add_f32 %[acc], %[acc], v69\n\t"
        "v_add_f32 %[acc], %[acc], v70\n\t"
        "v_add_f32 %[acc], %[acc], v71\n\t"
        "v_add_f32 %[acc], %[acc], v72\n\t"
        "v_add_f32 %[acc], %[acc], v73\n\t"
        "v_add_f32 %[acc], %[acc], v74\n\t"
        "v_add_f32 %[acc], %[acc], v75\n\t"
        "v_add_f32 %[acc], %[acc], v76\n\t"
        "v_add_f32 %[acc], %[acc], v77\n\t"
        "v_add_f32 %[acc], %[acc], v78\n\t"
        "v_add_f32 %[acc], %[acc], v79\n\t"
        "s_sub_u32 %[n], %[n], 1\n\t"
        "s_cmp_eq_u32 %[n], 0\n\t"
        "s_cbranch_scc1 2f\n\t"
        "s_waitcnt lgkmcnt(0)\n\t"
        "ds_read_b128 v[64:67], %[t] offset:128\n\t"
        "v_add_f32 %[acc], %[acc], v80\n\t"
        "ds_read_b128 v[68:71], %[t] offset:144\n\t"
        "v_add_f32 %[acc], %[acc], v81\n\t"
        "ds_read_b128 v[72:75], %[t] offset:160\n\t"
        "v_add_f32 %[acc], %[acc], v82\n\t"
        "ds_read_b128 v[76:79], %[t] offset:176\n\t"
        "v_add_f32 %[acc], %[acc], v83\n\t"
        "v_add_f32 %[acc], %[acc], v84\n\t"
        "v_add_f32 %[acc], %[acc], v85\n\t"
        "v_add_f32 %[acc], %[acc], v86\n\t"
        "v_add_f32 %[acc], %[acc], v87\n\t"
        "v_add_f32 %[acc], %[acc], v88\n\t"
        "v_add_f32 %[acc], %[acc], v89\n\t"
        "v_add_f32 %[acc], %[acc], v90\n\t"
        "v_add_f32 %[acc], %[acc], v91\n\t"
        "v_add_f32 %[acc], %[acc], v92\n\t"
        "v_add_f32 %[acc], %[acc], v93\n\t"
        "v_add_f32 %[acc], %[acc], v94\n\t"
        "v_add_f32 %[acc], %[acc], v95\n\t"
        "v_add_u32 %[t], 0x80, %[t]\n\t"
        "s_sub_u32 %[n], %[n], 1\n\t"
        "s_cmp_lg_u32 %[n], 0\n\t"
        "s_cbranch_scc1 1b\n\t"
        "2:\n\t"
        "s_waitcnt lgkmcnt(0)"
        : [acc] "+v"(acc), [t] "+v"(ta), [n] "+s"(n16)
        :
        : "v64", "v65", "v66", "v67", "v68", "v69", "v70", "v71", "v72", "v73", "v74", "v75", "v76", "v77", "v78", "v79", "v80", "v81", "v82", "v83", "v84", "v85", "v86", "v87", "v88", "v89", "v90", "v91", "v92", "v93", "v94", "v95", "scc", "memory");
  }
  const int done = n & ~15;
  float r[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) r[i] = t[done + i];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (done + i < n) acc = acc + r[i];
  return acc;
}

// acc = fma(w[k], v[k], acc) for k = 0 .. n - 1, in that order: w the weights and v this lane's
// row of values, both f32 in LDS, 16-byte aligned, 16 keys past n readable.
// Batches of 16 keys in assembly: per batch four 16-byte weight reads (the same address in every
// lane) and four 16-byte value reads, issued while the batch before is summed (weights
// v64-v79 / v96-v111, values v80-v95 / v112-v127 in turn); the rest in C++.
__device__ __forceinline__ float value_chain_lds(const float* w, const float* v, int n, float acc) {
  int n16 = __builtin_amdgcn_readfirstlane(n >> 4);
  uint32_t wa = lds_addr(w), va = lds_addr(v);
  if (n16 > 0) {
    {
      asm volatile(
          "ds_read_b128 v[64:67], %[w]\n\t"
          "ds_read_b128 v[68:71], %[w] offset:16\n\t"
          "ds_read_b128 v[72:75], %[w] offset:32\n\t"
          "ds_read_b128 v[76:79], %[w] offset:48\n\t"
          "ds_read_b128 v[80:83], %[v]\n\t"
          "ds_read_b128 v[84:87], %[v] offset:16\n\t"
          "ds_read_b128 v[88:91], %[v] offset:32\n\t"
          "ds_read_b128 v[92:95], %[v] offset:48\n\t"
          "v_add_u32 %[w], 64, %[w]\n\t"
          "v_add_u32 %[v], 64, %[v]\n\t"
          "1:\n\t"
          "s_waitcnt lgkmcnt(0)\n\t"
          "ds_read_b128 v[96:99], %[w]\n\t"
          "v_fmac_f32 %[acc], v64, v80\n\t"
          "v_fmac_f32 %[acc], v65, v81\n\t"
          "ds_read_b128 v[100:103], %[w] offset:16\n\t"
          "v_fmac_f32 %[acc], v66, v82\n\t"
          "v_fmac_f32 %[acc], v67, v83\n\t"
          "ds_read_b128 v[104:107], %[w] offset:32\n\t"
          "v_fmac_f32 %[acc], v68, v84\n\t"
          "v_fmac_f32 %[acc], v69, v85\n\t"
          "ds_read_b128 v[108:111], %[w] offset:48\n\t"
          "v_fmac_f32 %[acc], v70, v86\n\t"
          "v_fmac_f32 %[acc], v71, v87\n\t"
          "ds_read_b128 v[112:115], %[v]\n\t"
          "v_fmac_f32 %[acc], v72, v88\n\t"
          "v_fmac_f32 %[acc], v73, v89\n\t"
          "ds_read_b128 v[116:119], %[v] offset:16\n\t"
          "v_fmac_f32 %[acc], v74, v90\n\t"
          "v_fmac_f32 %[acc], v75, v91\n\t"
          "ds_read_b128 v[120:123], %[v] offset:32\n\t"
          "v_fmac_f32 %[acc], v76, v92\n\t"
          "v_fmac_f32 %[acc], v77, v93\n\t"
          "ds_read_b128 v[124:127], %[v] offset:48\n\t"
          "v_fmac_f32 %[acc], v78, v94\n\t"
          "v_fmac_f32 %[acc], v79, v95\n\t"
          "v_add_u32 %[w], 64, %[w]\n\t"
          "v_add_u32 %[v], 64, %[v]\n\t"
          "s_sub_u32 %[n], %[n], 1\n\t"
          "s_cmp_eq_u32 %[n], 0\n\t"
          "s_cbranch_scc1 2f\n\t"
          "s_waitcnt lgkmcnt(0)\n\t"
          "ds_read_b128 v[64:67], %[w]\n\t"
          "v_fmac_f32 %[acc], v96, v112\n\t"
          "v_fmac_f32 %[acc], v97, v113\n\t"
          "ds_read_b128 v[68:71], %[w] offset:16\n\t"
          "v_fmac_f32 %[acc], v98, v114\n\t"
          "v_fmac_f32 %[acc], v99, v115\n\t"
          "ds_read_b128 v[72:75], %[w] offset:32\n\t"
          "v_fmac_f32 %[acc], v100, v116\n\t"
          "v_fmac_f32 %[acc], v101, v117\n\t"
          "ds_read_b128 v[76:79], %[w] offset:48\n\t"
          "v_fmac_f32 %[acc], v102, v118\n\t"
          "v_fmac_f32 %[acc], v103, v119\n\t"
          "ds_read_b128 v[80:83], %[v]\n\t"
          "v_fmac_f32 %[acc], v104, v120\n\t"
          "v_fmac_f32 %[acc], v105, v121\n\t"
          "ds_read_b128 v[84:87], %[v] offset:16\n\t"
          "v_fmac_f32 %[acc], v106, v122\n\t"
          "v_fmac_f32 %[acc], v107, v123\n\t"
          "ds_read_b128 v[88:91], %[v] offset:32\n\t"
          "v_fmac_f32 %[acc], v108, v124\n\t"
          "v_fmac_f32 %[acc], v109, v125\n\t"
          "ds_read_b128 v[92:95], %[v] offset:48\n\t"
          "v_fmac_f32 %[acc], v110, v126\n\t"
          "v_fmac_f32 %[acc], v111, v127\n\t"
          "v_add_u32 %[w], 64, %[w]\n\t"
          "v_add_u32 %[v], 64, %[v]\n\t"
          "s_sub_u32 %[n], %[n], 1\n\t"
          "s_cmp_lg_u32 %[n], 0\n\t"
          "s_cbranch_scc1 1b\n\t"
          "2:\n\t"
          "s_waitcnt lgkmcnt(0)"
          : [acc] "+v"(acc), [w] "+v"(wa), [v] "+v"(va), [n] "+s"(n16)
          :
          : "v64", "v65", "v66", "v67", "v68", "v69", "v70", "v71", "v72", "v73", "v74", "v75", "v76", "v77", "v78", "v79", "v80", "v81", "v82", "v83", "v84", "v85", "v86", "v87", "v88", "v89", "v90", "v91", "v92", "v93", "v94", "v95", "v96", "v97", "v98", "v99", "v100", "v101", "v102", "v103", "v104", "v105", "v106", "v107", "v108", "v109", "v110", "v111", "v112", "v113", "v114", "v115", "v116", "v117", "v118", "v119", "v120", "v121", "v122", "v123", "v124", "v125", "v126", "v127", "scc", "memory");
    }
  }
  const int done = n & ~15;
  float wr[16], xr[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    wr[i] = w[done + i];
    xr[i] = v[done + i];
  }
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (done + i < n) acc = fmaf(wr[i], xr[i], acc);
  return acc;
}


constexpr unsigned kMeetSpinLimit = 1u << 22;

template <int HD, bool BF16KV, int S>
__device__ __forceinline__ void attn_split_unit(const AttnArgs& a, int hu, int j, const int* spos, uint64_t* scores,
                                                unsigned* abort_flag, unsigned char* smem, RowSync& rs) {
  constexpr int E = BF16KV ? 2 : 4;
  constexpr int C = HD / 16;
  constexpr int DS = HD / S;  // dims of this unit
  static_assert(HD % S == 0, "split of the head dims");
  const int cap = a.cap, H = a.H, KVH = a.KVH;
  const float scale = a.scale;
  const unsigned tag = a.split_tag;
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
  uint64_t* srow = scores + (size_t)hu * cap;
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
    if (li == 0 && k < k1) st_co(srow + k, (uint64_t)tag << 32 | __float_as_uint(scale * (acc + 0.0f)));
    if (li == 0 && k + 32 < k1) st_co(srow + k + 32, (uint64_t)tag << 32 | __float_as_uint(scale * (acz + 0.0f)));
  }
  // ---- V columns [j DS, (j + 1) DS) of keys 0 .. L - 1: waves 4 .. 7 stage them as [key][DS]
  // by direct loads of PB-byte pieces (piece pc = key PPK + part; a piece past the last repeats
  // it) and later turn their own pieces into the rows; waves 0 .. 3 meanwhile read the scores
  constexpr int PB = split_piece_bytes(HD, BF16KV ? 1 : 0, S), PPK = DS * E / PB;
  const int lp = split_row_words(cap), np = L * PPK;
  float* vt = (float*)smem;
  unsigned char* stage = smem + split_rows_bytes(cap, HD, S);
  float* w = (float*)(stage + split_stage_bytes(cap, HD, BF16KV ? 1 : 0, S));
  float* slot = w + cap + kSplitSlack;  // [0, 8): wave maxima; [8, 16): waves whose wait gave up; 16: the sum
  float mx = -__builtin_huge_valf();
  int ok = 1;
  if (wave >= 4) {
    const unsigned char* vc = (const unsigned char*)a.vc;
    for (int r = 0; r * 256 < np; ++r) {
      const int pc = min(r * 256 + (wave - 4) * kWave + lane, np - 1);
      const int key = pc / PPK, part = pc % PPK;
      lds_dma<PB, false>(vc + ((base + (size_t)((first + key) % cap)) * HD + j * DS) * E + part * PB,
                         stage + (size_t)(r * 256 + (wave - 4) * kWave) * PB);
    }
  } else {
    // ---- the head's scores, each entry read until it carries this launch's tag
    for (int k0r = threadIdx.x; k0r < L; k0r += 4 * 256) {
      uint64_t e[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) e[u] = ld_co(srow + min(k0r + u * 256, L - 1));
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int k = k0r + u * 256;
        if (k >= L) break;
        unsigned spins = 0;
        while ((unsigned)(e[u] >> 32) != tag && ok) {
          if (++spins > kMeetSpinLimit) {
            __hip_atomic_store(gbl(abort_flag), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ok = 0;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
          e[u] = ld_co(srow + k);
        }
        const float v = __uint_as_float((uint32_t)e[u]);
        w[k] = v;
        mx = fmaxf(mx, v);
      }
    }
  }
  const int failed = __any(!ok) ? 1 : 0;
  mx = wave_max(mx);
  if (lane == 0) {
    slot[wave] = mx;
    ((int*)slot)[8 + wave] = failed;
  }
  rs.sync();
  int any_failed = 0;
#pragma unroll
  for (int i = 0; i < kRowWaves; ++i) any_failed |= ((const int*)slot)[8 + i];
  if (any_failed) {
    __builtin_amdgcn_s_waitcnt(kVmWait0);  // the direct loads have landed before the wave ends
    return;
  }
  // ---- softmax over the head's L scores, every unit of the head alike
  mx = slot[0];
#pragma unroll
  for (int i = 1; i < kRowWaves; ++i) mx = fmaxf(mx, slot[i]);
  for (int k = threadIdx.x; k < L; k += kRowThreads) w[k] = ref_exp(w[k] - mx);
  rs.sync();
  if (threadIdx.x == 0) {
    slot[16] = ordered_sum_lds(w, L, 0.0f);
  } else if (wave >= 4) {
    // the staged pieces of this wave into the rows (bf16 widened), while thread 0 sums
    __builtin_amdgcn_s_waitcnt(kVmWait0);
    for (int pc = (wave - 4) * kWave + lane; pc < np; pc += 256) {
      const int key = pc / PPK, d0 = pc % PPK * (PB / E);
      const unsigned char* src = stage + (size_t)pc * PB;
      if constexpr (PB == 16) {
        const uint4 x = *(const uint4*)src;
        const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (BF16KV) {
            vt[(size_t)(d0 + 2 * i) * lp + key] = __uint_as_float(xs[i] << 16);
            vt[(size_t)(d0 + 2 * i + 1) * lp + key] = __uint_as_float(xs[i] & 0xffff0000u);
          } else {
            vt[(size_t)(d0 + i) * lp + key] = __uint_as_float(xs[i]);
          }
        }
      } else {
        const uint32_t x = *(const uint32_t*)src;
        if constexpr (BF16KV) {
          vt[(size_t)d0 * lp + key] = __uint_as_float(x << 16);
          vt[(size_t)(d0 + 1) * lp + key] = __uint_as_float(x & 0xffff0000u);
        } else {
          vt[(size_t)d0 * lp + key] = __uint_as_float(x);
        }
      }
    }
  }
  rs.sync();
  const float sum = slot[16];
  for (int k = threadIdx.x; k < L; k += kRowThreads) w[k] = w[k] / sum;
  rs.sync();
  // ---- out_d = mul_add(w_k, v_kd, out_d) over keys in order: lane d of wave 0 owns dim j DS + d
  if (wave != 0 || lane >= DS) return;
  const float acc = value_chain_lds(w, vt + (size_t)lane * lp, L, 0.0f);
  st_co(a.out + (size_t)b * H * HD + (size_t)h * HD + j * DS + lane, acc);
}

}  // namespace

// Launched with the row waves only.  Units u < hheads map to (head hu, part j); with a multiple
// of 8 heads the S units of a head share u % 8, and with it the XCD that dispatch places them on
// (whose L2 then serves the V rows that all of them read).  Units past `hheads` gather the next
// step's audio embedding rows (the first attention phase of an STT step).
template <int AV, int S>
__global__ __launch_bounds__(kRowThreads) void attn_split_kernel(const float* hq, const void* hkc, const void* hvc,
                                                                 const int* hpos, uint64_t* hscores, int hcap, int hwindow,
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

using SplitKernel = void (*)(const float*, const void*, const void*, const int*, uint64_t*, int, int, int, int, const Phase,
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

hipError_t launch_attn_split(const Phase& ph, const StepParams& p, int step, int S, uint64_t* scores, hipStream_t s) {
  const AttnArgs& a = ph.at;
  const int hd = a.hd == 128 ? 128 : 64;
  if (a.hd != hd || !scores) return hipErrorInvalidValue;
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
