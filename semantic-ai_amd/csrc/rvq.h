// Mimi's split residual vector quantizer, encoding (SVL/stt/model.rs:84-174), on the GPU.
//
// Codebook stage s < n_q holds `bins` entries of kRvqDim f32 (stage 0: the first quantizer's
// codebook; stages 1 .. n_q - 1: the rest quantizer's codebooks in order) and their half norms.
// A call encodes `rows` latent vectors (kRvqIn channels each, read channel-first with a stride of
// `frames` from [batch][kRvqIn][frames]).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace svl {

constexpr int kRvqIn = 512;   // latent channels
constexpr int kRvqDim = 256;  // codebook dims (ResidualQuantizer::DIM)
constexpr int kRvqBlock = 64; // codebook entries per workgroup of a stage
constexpr int kRvqTile = 32;  // rows per workgroup of a stage

// embedding = sums / max(usage, 1e-5); half norms = (sum of squares in dim order) * 0.5 + 0
// (Codebook::new, SVL/stt/model.rs:144-153), for `entries` entries.
hipError_t launch_rvq_prepare(const float* sums, const float* usage, size_t entries, float* emb, float* hn,
                              hipStream_t s);
// proj[part][row][o] = 16-lane dot of input_proj row o of part (0: first, 1: rest) with the row's
// latents (ResidualQuantizer::encode's 1x1 convolution, SVL/stt/model.rs:126).
hipError_t launch_rvq_project(const float* latents, int batch, int frames, const float* w_first, const float* w_rest,
                              float* proj, hipStream_t s);
// Stage k of the rest chain (and, for k = 0, the first chain's only stage): the residual of every
// row (k = 0: its projection; then the previous residual minus the entry that stage chose), kept
// in res[k % 2] for the next stage, then for every entry the score half_norm - residual . entry
// and the per-row minimum (score, then index) into keys[stage][row].
hipError_t launch_rvq_stage(int k, int n_q, int rows, int bins, const float* emb, const float* hn, const float* proj,
                            float* res, unsigned long long* keys, hipStream_t s);
// codes[row][q] = the index in keys[q][row].
hipError_t launch_rvq_codes(const unsigned long long* keys, int rows, int n_q, uint32_t* codes, hipStream_t s);

}  // namespace svl
