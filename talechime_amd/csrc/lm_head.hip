// lm_head.hip -- the LM head that feeds the sampler, and the two in one call.
//
// The step before the sampler in talechime's AR loops is a Linear layer over
// the last hidden state: indextts's mel_head (1280 -> 8194 with a bias,
// crates/indextts/src/generation.rs:632, 981), the qwen3-tts code predictor's
// lm_heads (hidden -> 2048 without one, crates/qwen3-tts/src/models/
// code_predictor.rs:208-216), the talker's codec_head.  At decode sizes (a few
// rows) it is a matrix-vector product bound by reading the weight matrix:
// 21 MB of bf16 at 1280 x 8194, 2.6 us at 8 TB/s.  There is no contraction
// deep enough for MFMA to pay (each weight is used by <= 4 rows per pass), so
// the kernel streams the weights once per group of rows with 16-byte loads
// and accumulates in f32 on the VALU.
//
// k_lm_head_reg (up to 4 rows, the decode case): one wave per block of
// kHeadVB vocabulary rows; lane l takes the 16-byte chunks l, l + 64, ... of
// each weight row and the matching slices of the hidden rows, loaded first so
// that they are in when the weights arrive; no LDS and no barrier.
// k_lm_head (more rows): the same weight layout held in registers while the
// hidden rows pass through LDS kHeadRG8 at a time, so the weights are read
// once whatever the number of rows.  Each lane keeps kHeadVB x rows partial
// dot products, reduced across the wave with DPP at the end.  Logit = that
// dot product + bias (candle's Linear: matmul, then broadcast add), the bias
// loaded with the weights.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/talechime_hip.h"
#include "tc_dpp.h"

namespace tc {

constexpr int kHeadVB = 4;      // vocabulary rows per wave
constexpr int kHeadRG = 4;      // hidden rows per LDS chunk when 8 do not fit
constexpr int kHeadRG8 = 8;     // hidden rows per LDS chunk
constexpr size_t kHeadLds = 64 * 1024;  // dynamic LDS per workgroup at most
constexpr int kHeadCPL = 8;     // 16-byte weight chunks per lane at most (bf16: dim <= 4096)
constexpr int kHeadWaves = 4;   // waves per workgroup
constexpr int kHeadMaxDim = 4096;

// The library's error slot (tc_last_error), set by the entry points below.
int set_error(int code, const char* msg);

struct HeadArgs {
  const float* hidden;  // [rows, hid_ld] f32, rows <= kHeadRG in this pass
  long long hid_ld;
  const void* weight;   // [vocab, dim], f32 or bf16, row stride dim
  const float* bias;    // [vocab] or null
  float* logits;        // [rows, out_ld]
  long long out_ld;
  int rows, dim, vocab;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// CPL: the 16-byte chunks per lane the launch needs (dim / elements per
// chunk / 64, rounded up); the hidden rows take kHeadRG * dim floats of
// dynamic LDS.
template <typename WT, int CPL, int RG>
__global__ void __launch_bounds__(kHeadWaves * 64) k_lm_head(HeadArgs a) {
  extern __shared__ __align__(16) float hs[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int kEpc = sizeof(WT) == 2 ? 8 : 4;  // elements per 16-byte chunk
  const int nchunk = a.dim / kEpc;
  const int v0 = (blockIdx.x * kHeadWaves + wave) * kHeadVB;
  // the wave's bias values and every weight chunk of its rows, issued first
  // so that HBM works while the hidden rows are staged
  float bsv[kHeadVB];
#pragma unroll
  for (int b = 0; b < kHeadVB; ++b) bsv[b] = a.bias ? a.bias[min(v0 + b, a.vocab - 1)] : 0.0f;
  uint4 w[kHeadVB][CPL];
#pragma unroll
  for (int b = 0; b < kHeadVB; ++b) {
    const int v = min(v0 + b, a.vocab - 1);
    const uint4* row = reinterpret_cast<const uint4*>(reinterpret_cast<const WT*>(a.weight) + (size_t)v * (size_t)a.dim);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      w[b][j] = (c < nchunk && v0 < a.vocab) ? row[c] : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  // the rows RG at a time through LDS while the weights stay in registers:
  // HBM reads the weights once whatever the number of rows (rows past
  // a.rows read as zeros; dim is a multiple of 4)
  const int q4 = a.dim >> 2;
  for (int r0 = 0; r0 < a.rows; r0 += RG) {
    for (int i = threadIdx.x; i < RG * q4; i += blockDim.x) {
      const int r = i / q4, k = i - r * q4;
      float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (r0 + r < a.rows) v = reinterpret_cast<const float4*>(a.hidden + (size_t)(r0 + r) * (size_t)a.hid_ld)[k];
      reinterpret_cast<float4*>(hs)[i] = v;
    }
    __syncthreads();
    if (v0 < a.vocab) {
      float acc[kHeadVB][RG];
#pragma unroll
      for (int b = 0; b < kHeadVB; ++b)
#pragma unroll
        for (int r = 0; r < RG; ++r) acc[b][r] = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        if (c >= nchunk) break;
        // the chunk's weights widened once, then one pass over the hidden rows
        float wf[kHeadVB][8];
#pragma unroll
        for (int b = 0; b < kHeadVB; ++b) {
          const uint4 q = w[b][j];
          if (kEpc == 8) {
            wf[b][0] = bf16_lo(q.x); wf[b][1] = bf16_hi(q.x); wf[b][2] = bf16_lo(q.y); wf[b][3] = bf16_hi(q.y);
            wf[b][4] = bf16_lo(q.z); wf[b][5] = bf16_hi(q.z); wf[b][6] = bf16_lo(q.w); wf[b][7] = bf16_hi(q.w);
          } else {
            wf[b][0] = __uint_as_float(q.x); wf[b][1] = __uint_as_float(q.y);
            wf[b][2] = __uint_as_float(q.z); wf[b][3] = __uint_as_float(q.w);
          }
        }
#pragma unroll
        for (int r = 0; r < RG; ++r) {
          float h[8];
          const float4* hp = reinterpret_cast<const float4*>(&hs[r * a.dim + c * kEpc]);
          const float4 h0 = hp[0];
          h[0] = h0.x; h[1] = h0.y; h[2] = h0.z; h[3] = h0.w;
          if (kEpc == 8) {
            const float4 h1 = hp[1];
            h[4] = h1.x; h[5] = h1.y; h[6] = h1.z; h[7] = h1.w;
          }
#pragma unroll
          for (int b = 0; b < kHeadVB; ++b) {
            float s = acc[b][r];
#pragma unroll
            for (int e = 0; e < kEpc; ++e) s = __builtin_fmaf(wf[b][e], h[e], s);
            acc[b][r] = s;
          }
        }
      }
#pragma unroll
      for (int b = 0; b < kHeadVB; ++b) {
        const int v = v0 + b;
#pragma unroll
        for (int r = 0; r < RG; ++r) {
          const float t = dpp_wave_sum(acc[b][r]);
          if (lane == 0 && v < a.vocab && r0 + r < a.rows)
            a.logits[(size_t)(r0 + r) * (size_t)a.out_ld + v] = a.bias ? t + bsv[b] : t;
        }
      }
    }
    __syncthreads();  // every wave is done with this chunk's rows
  }
}

// Decode sizes (rows per pass x chunks per lane <= kHeadRegSlices): no LDS and
// no barrier.  Each lane loads the slices of the hidden rows its chunks meet
// (chunk c covers elements kEpc c .. kEpc c + kEpc - 1 of every row), then
// every weight chunk of the wave's rows, chunk by chunk: the loads return in
// issue order, so the products of chunk j start as soon as its weights are in
// while the later chunks are still on their way.  The hidden rows come from
// L2 after the first waves read them.
constexpr int kHeadRegSlices = 12;
template <typename WT, int CPL, int RG>
__global__ void __launch_bounds__(kHeadWaves * 64) k_lm_head_reg(HeadArgs a) {
  static_assert(CPL * RG <= kHeadRegSlices, "hidden slices held per lane");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int kEpc = sizeof(WT) == 2 ? 8 : 4;  // elements per 16-byte chunk
  constexpr int kHq = kEpc / 4;                   // float4 of hidden values per chunk
  const int nchunk = a.dim / kEpc;
  const int v0 = (blockIdx.x * kHeadWaves + wave) * kHeadVB;
  if (v0 >= a.vocab) return;
  // the wave's bias values, in flight with everything else
  float bsv[kHeadVB];
#pragma unroll
  for (int b = 0; b < kHeadVB; ++b) bsv[b] = a.bias ? a.bias[min(v0 + b, a.vocab - 1)] : 0.0f;
  float4 hv[CPL][RG][kHq];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const float4* hp = reinterpret_cast<const float4*>(a.hidden + (size_t)r * (size_t)a.hid_ld) + c * kHq;
#pragma unroll
      for (int q = 0; q < kHq; ++q)
        hv[j][r][q] = (c < nchunk && r < a.rows) ? hp[q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  }
  uint4 w[CPL][kHeadVB];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
#pragma unroll
    for (int b = 0; b < kHeadVB; ++b) {
      const int v = min(v0 + b, a.vocab - 1);
      const uint4* row = reinterpret_cast<const uint4*>(reinterpret_cast<const WT*>(a.weight) + (size_t)v * (size_t)a.dim);
      w[j][b] = c < nchunk ? row[c] : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  float acc[kHeadVB][RG];
#pragma unroll
  for (int b = 0; b < kHeadVB; ++b)
#pragma unroll
    for (int r = 0; r < RG; ++r) acc[b][r] = 0.0f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    if (lane + 64 * j >= nchunk) break;
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      float h[8];
      h[0] = hv[j][r][0].x; h[1] = hv[j][r][0].y; h[2] = hv[j][r][0].z; h[3] = hv[j][r][0].w;
      if (kEpc == 8) {
        h[4] = hv[j][r][kHq - 1].x; h[5] = hv[j][r][kHq - 1].y; h[6] = hv[j][r][kHq - 1].z; h[7] = hv[j][r][kHq - 1].w;
      }
#pragma unroll
      for (int b = 0; b < kHeadVB; ++b) {
        const uint4 q = w[j][b];
        float s = acc[b][r];
        if (kEpc == 8) {
          s = __builtin_fmaf(bf16_lo(q.x), h[0], s);
          s = __builtin_fmaf(bf16_hi(q.x), h[1], s);
          s = __builtin_fmaf(bf16_lo(q.y), h[2], s);
          s = __builtin_fmaf(bf16_hi(q.y), h[3], s);
          s = __builtin_fmaf(bf16_lo(q.z), h[4], s);
          s = __builtin_fmaf(bf16_hi(q.z), h[5], s);
          s = __builtin_fmaf(bf16_lo(q.w), h[6], s);
          s = __builtin_fmaf(bf16_hi(q.w), h[7], s);
        } else {
          s = __builtin_fmaf(__uint_as_float(q.x), h[0], s);
          s = __builtin_fmaf(__uint_as_float(q.y), h[1], s);
          s = __builtin_fmaf(__uint_as_float(q.z), h[2], s);
          s = __builtin_fmaf(__uint_as_float(q.w), h[3], s);
        }
        acc[b][r] = s;
      }
    }
  }
#pragma unroll
  for (int b = 0; b < kHeadVB; ++b) {
    const int v = v0 + b;
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const float t = dpp_wave_sum(acc[b][r]);
      if (lane == 0 && v < a.vocab && r < a.rows)
        a.logits[(size_t)r * (size_t)a.out_ld + v] = a.bias ? t + bsv[b] : t;
    }
  }
}

}  // namespace tc

namespace {
int head_fail(int code, const char* msg) { return tc::set_error(code, msg); }

// The register kernel for rg rows per pass (1..4) and cpl chunks per lane,
// when rg x cpl fits its hidden slices; false otherwise.
template <typename WT, int RG>
bool launch_head_reg_rg(int cpl, unsigned blocks, hipStream_t st, const tc::HeadArgs& a, hipError_t* e) {
  const dim3 g(blocks), b(tc::kHeadWaves * 64);
  constexpr int kMax = tc::kHeadRegSlices / RG;
  if (cpl <= 1) hipLaunchKernelGGL((tc::k_lm_head_reg<WT, 1, RG>), g, b, 0, st, a);
  else if (cpl <= 2 && kMax >= 2) hipLaunchKernelGGL((tc::k_lm_head_reg<WT, (kMax >= 2 ? 2 : 1), RG>), g, b, 0, st, a);
  else if (cpl <= 3 && kMax >= 3) hipLaunchKernelGGL((tc::k_lm_head_reg<WT, (kMax >= 3 ? 3 : 1), RG>), g, b, 0, st, a);
  else if (cpl <= 4 && kMax >= 4) hipLaunchKernelGGL((tc::k_lm_head_reg<WT, (kMax >= 4 ? 4 : 1), RG>), g, b, 0, st, a);
  else if (cpl <= 8 && kMax >= 8) hipLaunchKernelGGL((tc::k_lm_head_reg<WT, (kMax >= 8 ? 8 : 1), RG>), g, b, 0, st, a);
  else return false;
  *e = hipGetLastError();
  return true;
}
template <typename WT>
bool launch_head_reg(int rows, int cpl, unsigned blocks, hipStream_t st, const tc::HeadArgs& a, hipError_t* e) {
  if (rows <= 1) return launch_head_reg_rg<WT, 1>(cpl, blocks, st, a, e);
  if (rows <= 2) return launch_head_reg_rg<WT, 2>(cpl, blocks, st, a, e);
  if (rows <= 3) return launch_head_reg_rg<WT, 3>(cpl, blocks, st, a, e);
  if (rows <= 4) return launch_head_reg_rg<WT, 4>(cpl, blocks, st, a, e);
  return false;
}

template <typename WT, int CPL, int RG>
hipError_t launch_head_k(unsigned blocks, size_t lds, hipStream_t st, const tc::HeadArgs& a) {
  hipLaunchKernelGGL((tc::k_lm_head<WT, CPL, RG>), dim3(blocks), dim3(tc::kHeadWaves * 64), lds, st, a);
  return hipGetLastError();
}
template <typename WT, int RG>
hipError_t launch_head_rg(int cpl, unsigned blocks, size_t lds, hipStream_t st, const tc::HeadArgs& a) {
  if (cpl <= 1) return launch_head_k<WT, 1, RG>(blocks, lds, st, a);
  if (cpl <= 2) return launch_head_k<WT, 2, RG>(blocks, lds, st, a);
  if (cpl <= 3) return launch_head_k<WT, 3, RG>(blocks, lds, st, a);
  if (cpl <= 4) return launch_head_k<WT, 4, RG>(blocks, lds, st, a);
  return launch_head_k<WT, 8, RG>(blocks, lds, st, a);
}
template <typename WT>
hipError_t launch_head(int rg, int cpl, unsigned blocks, size_t lds, hipStream_t st, const tc::HeadArgs& a) {
  if (rg == tc::kHeadRG8) return launch_head_rg<WT, tc::kHeadRG8>(cpl, blocks, lds, st, a);
  return launch_head_rg<WT, tc::kHeadRG>(cpl, blocks, lds, st, a);
}
}  // namespace

extern "C" {

int tc_lm_head(const float* d_hidden, size_t hidden_ld, const void* d_weight, int w_dtype, const float* d_bias,
               size_t rows, size_t dim, size_t vocab, float* d_logits, size_t logits_ld, tc_stream stream) {
  if (rows == 0) return TC_OK;
  if (!d_hidden || !d_weight || !d_logits) return head_fail(TC_EINVAL, "tc_lm_head: NULL device pointer");
  if (w_dtype != TC_F32 && w_dtype != TC_BF16) return head_fail(TC_EINVAL, "tc_lm_head: weight dtype");
  const size_t epc = w_dtype == TC_BF16 ? 8 : 4;
  if (dim == 0 || dim % epc || dim > (size_t)tc::kHeadMaxDim || dim / epc > (size_t)(64 * tc::kHeadCPL))
    return head_fail(TC_EUNSUPPORTED, "tc_lm_head: dim must be a multiple of 8 (bf16) or 4 (f32), at most 4096 "
                                      "(bf16) or 2048 (f32)");
  if (vocab == 0 || vocab > (size_t)INT32_MAX || hidden_ld < dim || logits_ld < vocab)
    return head_fail(TC_EINVAL, "tc_lm_head: shape");
  if (reinterpret_cast<uintptr_t>(d_weight) & 15u) return head_fail(TC_EINVAL, "tc_lm_head: weight not 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(d_hidden) & 15u) || hidden_ld % 4)
    return head_fail(TC_EINVAL, "tc_lm_head: hidden rows must be 16-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const unsigned blocks = (unsigned)((vocab + tc::kHeadVB * tc::kHeadWaves - 1) / (tc::kHeadVB * tc::kHeadWaves));
  const int cpl = (int)((dim / epc + 63) / 64);
  // the register kernel when every row fits its hidden slices in one pass
  // (up to 4 rows); more rows take the LDS kernel, whose passes hold 8 or 16
  const int cpl_t = cpl <= 4 ? cpl : 8;  // the kernels' chunk counts: 1, 2, 3, 4, 8
  const int reg_rg = tc::kHeadRegSlices / cpl_t < 4 ? tc::kHeadRegSlices / cpl_t : 4;
  if (reg_rg >= 1 && rows <= (size_t)reg_rg) {
    for (size_t r0 = 0; r0 < rows; r0 += (size_t)reg_rg) {
      tc::HeadArgs a{};
      a.hidden = d_hidden + r0 * hidden_ld;
      a.hid_ld = (long long)hidden_ld;
      a.weight = d_weight;
      a.bias = d_bias;
      a.logits = d_logits + r0 * logits_ld;
      a.out_ld = (long long)logits_ld;
      a.rows = (int)(rows - r0 < (size_t)reg_rg ? rows - r0 : (size_t)reg_rg);
      a.dim = (int)dim;
      a.vocab = (int)vocab;
      hipError_t e = hipSuccess;
      const bool ok = w_dtype == TC_BF16 ? launch_head_reg<uint16_t>(a.rows, cpl, blocks, st, a, &e)
                                         : launch_head_reg<float>(a.rows, cpl, blocks, st, a, &e);
      if (!ok) return head_fail(TC_EHIP, "tc_lm_head: no register kernel for this shape");
      if (e != hipSuccess) return head_fail(TC_EHIP, hipGetErrorString(e));
    }
    return TC_OK;
  }
  // one launch for every row: the kernel takes them 8 (or, past the LDS, 4)
  // at a time through LDS with the weights held in registers
  const int rg = (size_t)tc::kHeadRG8 * dim * sizeof(float) <= tc::kHeadLds ? tc::kHeadRG8 : tc::kHeadRG;
  const size_t lds = (size_t)rg * dim * sizeof(float);
  tc::HeadArgs a{};
  a.hidden = d_hidden;
  a.hid_ld = (long long)hidden_ld;
  a.weight = d_weight;
  a.bias = d_bias;
  a.logits = d_logits;
  a.out_ld = (long long)logits_ld;
  a.rows = (int)rows;
  a.dim = (int)dim;
  a.vocab = (int)vocab;
  const hipError_t e = w_dtype == TC_BF16 ? launch_head<uint16_t>(rg, cpl, blocks, lds, st, a)
                                          : launch_head<float>(rg, cpl, blocks, lds, st, a);
  if (e != hipSuccess) return head_fail(TC_EHIP, hipGetErrorString(e));
  return TC_OK;
}

int tc_head_sample(tc_ctx* ctx, const tc_sample_params* params, const float* d_hidden, size_t hidden_ld,
                   const void* d_weight, int w_dtype, const float* d_bias, size_t rows, size_t dim, size_t vocab,
                   float* d_logits, const uint32_t* d_hist_off, const uint32_t* d_hist_ids,
                   const void* d_uniforms, uint32_t* d_out_ids, int32_t* d_out_status, uint32_t* d_out_flags,
                   tc_stream stream) {
  int rc = tc_lm_head(d_hidden, hidden_ld, d_weight, w_dtype, d_bias, rows, dim, vocab, d_logits, vocab, stream);
  if (rc != TC_OK) return rc;
  return tc_sample(ctx, params, d_logits, TC_F32, rows, vocab, vocab, d_hist_off, d_hist_ids, d_uniforms, d_out_ids,
                   d_out_status, d_out_flags, nullptr, stream);
}

}  // extern "C"
