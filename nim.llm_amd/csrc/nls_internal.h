// nls_internal.h -- layouts shared by the host side (nls_api.cpp) and the
// gfx950 kernels (nls_kernels.hip).  Not part of the public ABI.
#pragma once
#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

namespace nls {

// Row modes, decided on the host from the row's SamplerParams
// (src/nimllm/sampler.nim:77-97).
enum RowMode : int32_t {
  kModeGreedy = 1,  // temperature <= 0: argmax (:77-78)
  kModeTopK = 2,    // 0 < k < V: heap path (:86-95)
  kModeFull = 3,    // k == 0 or k >= V: full stable sort path (:96-97)
};

// Per-row constants, precomputed on the host in the reference's precisions.
struct RowParams {
  float invT;     // float32(1.0 / temperature) (:80)
  float rp32;     // float32(repeatPenalty) (:72-73)
  float minP32;   // float32(minP) (:111)
  int32_t mode;   // RowMode
  int32_t k;      // effective k (:85); V on the full path
  int32_t pen_active;  // rp != 1 or presence != 0 or frequency != 0 (:64-65)
  int32_t rp_active;   // rp != 1 (:71)
  int32_t topp_active; // 0 < topP < 1 (:103)
  int32_t minp_active; // minP > 0 (:110)
  int32_t bias_off;    // into the per-handle bias arrays (sorted, unique, in range)
  int32_t bias_cnt;
  int32_t fast;        // 1: top-k row handled by the chunk+merge kernels
  double topP;         // compared in float64 (:107)
  double freq;         // frequencyPenalty
  double pres;         // presencePenalty
  int64_t repeat_last_n;
};

// One logit touched by penalties and/or bias; the per-row list is sorted by id.
enum PatchFlags : int32_t { kPatchPen = 1, kPatchBias = 2 };
struct Patch {
  int32_t id;
  int32_t flags;
  float pen;   // float32(cnt * frequency + presence), formed in float64 (:74)
  float bias;  // float32(logitBias[id]) (:76)
};

// Per (row, chunk) summary written by the streaming pass.
enum ChunkFlags : int32_t { kChunkOverflow = 1 };
struct ChunkStat {
  float vmax;     // max of the chunk's final values (first index on ties)
  int32_t amax;   // its index (global token id)
  int32_t ncand;  // candidates written (top-k rows)
  int32_t flags;
};

// Streaming-pass geometry.
constexpr int kChunkThreads = 256;
constexpr int kChunkVec4 = 16;  // float4 loads per thread
constexpr int kChunkElems = kChunkThreads * kChunkVec4 * 4;  // 16384
constexpr int kMaxChunks = 64;
constexpr int kMaxTopKFast = 2048;   // larger k goes to the whole-row kernel
constexpr int kPrepSortLds = 4096;   // history+bias entries sorted in LDS
constexpr int kMergeThreads = 256;
constexpr int kGenericThreads = 1024;

inline int chunk_cap_for_k(int k) { return k + k / 4 + 64; }

struct DebugPtrs {
  int32_t* n;
  int32_t* ncand;
  int32_t* cand_ids;
  float* cand_probs;
  float* total;
  int32_t* path;
  int32_t cap;
};

struct LaunchArgs {
  const float* logits;
  int64_t V;
  int B;
  int nchunks;
  int qmax;  // max top-Q over top-k rows (1, 2, 4 or 8); 0 if none
  bool vec4;
  const RowParams* rp;
  const int32_t* hist;
  const int64_t* hist_len;
  int hcap;
  const int32_t* bias_ids;
  const float* bias_vals;
  Patch* patches;
  int32_t* patch_cnt;
  int pcap;
  uint64_t* prep_scratch;
  int64_t prep_stride;
  ChunkStat* stats;
  uint64_t* cand;
  int ccap;
  int mcap;
  size_t merge_lds;
  const double* d_u;
  uint64_t* rng;
  int32_t* out;
  float* row_max;
  int32_t* generic_list;
  int32_t* generic_count;
  uint32_t* gen_scratch;
  int64_t gen_vpad;
  int gen_blocks;
  DebugPtrs dbg;
  hipEvent_t ev_start;  // optional: recorded around the streaming kernel
  hipEvent_t ev_stop;
};

hipError_t launch_sample(const LaunchArgs& a, hipStream_t s);
hipError_t launch_accept_host(const int32_t* d_ids, int B, int count, int32_t* hist,
                              int64_t* hist_len, int hcap, int row_only, hipStream_t s);
hipError_t launch_accept_device(const int32_t* d_ids, int B, int64_t V, int32_t* hist,
                                int64_t* hist_len, int hcap, hipStream_t s);
hipError_t launch_expf(const float* x, float* y, int64_t n, hipStream_t s);
hipError_t set_kernel_attributes();

}  // namespace nls
