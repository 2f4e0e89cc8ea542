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
  int32_t fast;        // 1: greedy/top-k row handled by the streaming kernel
  double topP;         // compared in float64 (:107)
  double freq;         // frequencyPenalty
  double pres;         // presencePenalty
  int64_t repeat_last_n;
};

// Patch flags: which of penalty (:71-74) and bias (:76) touch a logit; in the
// streaming kernel also whether its original logit was met above the
// threshold (seen) and whether its patch can raise it (a positive or NaN
// bias).  The streaming kernel keeps the window count above the flag bits
// (a count > 0 means the penalty applies) instead of kPatchPen.
enum PatchFlags : uint32_t { kPatchPen = 1u, kPatchBias = 2u, kPatchSeen = 4u, kPatchRise = 8u };
constexpr int kPatchCountShift = 4;

// Streaming-kernel geometry.
constexpr int kStreamVec4 = 4;       // float4 loads per thread per tile
constexpr int kMaxTopKFast = 2048;   // larger k goes to the whole-row kernel
constexpr int kGenericThreads = 1024;
constexpr int kMaxSlices = 64;
constexpr int kWaveCap = 256;        // per-wave candidate buffer of the k <= 64 path
constexpr int kWaveTopK = 64;        // largest k of the wave path
constexpr size_t kDualStreamLds = 68 * 1024;  // dynamic LDS of a 512-thread workgroup, two per CU
constexpr int64_t kSmallRowV = 49152;  // rows up to this size stream in one workgroup

// k64_kernel (greedy and top-k <= 64 rows, one 1024-thread workgroup per
// row): LDS = patch bitmap | hash table (4 words per slot) | per-wave
// candidate buffers | bootstrap histogram (later the candidate list) | list
// of patched slots to evaluate.
constexpr int kK64Threads = 1024;
constexpr int kK64BootBins = 4096;
constexpr size_t kK64BootBytes = (size_t)kK64BootBins * 4;
constexpr int kK64CandCap = (int)(kK64BootBytes / 8);
constexpr int kK64PListCap = 1024;
constexpr int kK64MaxHash = 4096;
constexpr int kK64SelRegs = 4;  // candidates per lane of the register select (256 per row)
constexpr size_t kK64MaxDynLds = 138 * 1024;  // 160 KB of LDS less the kernel's static part
constexpr int kK64RankCap = 256;  // candidates ranked by the whole workgroup at the end
inline size_t k64_lds_bytes(int64_t V, int hbits) {
  const size_t nw = (size_t)((V + 31) / 32);
  return ((nw * 4 + 15) & ~(size_t)15) + ((size_t)16 << hbits) + (size_t)(kK64Threads / 64) * kWaveCap * 8 +
         kK64BootBytes + (size_t)kK64PListCap * 4;
}

// Slice-exchange record of one (row, slice) when a row is split over S
// workgroups.
enum SliceFlags : int32_t { kSliceOverflow = 1, kSliceNan0 = 2 /* element 0 of the row is NaN */ };
struct SliceInfo {
  int32_t n;      // candidates written
  int32_t flags;  // SliceFlags
  int32_t amax;   // first argmax of the slice's final values
  int32_t vmax;   // its value (float bits)
};

struct DebugPtrs {
  int32_t* n;
  int32_t* ncand;
  int32_t* cand_ids;
  float* cand_probs;
  float* total;
  int32_t* path;
  int32_t cap;
};

// OR-ed into a sampling row's debug path code when a NaN is among the row's
// candidates.  The key map orders a NaN with the sign bit clear above +inf
// (always a candidate) and one with it set below -inf; the reference's heap
// and sort comparisons (src/nimllm/sampler.nim:88-97) leave a row with any
// NaN order-dependent, so such a row's result is this sampler's own.
constexpr int32_t kPathNaN = 0x100;

// Grouped sort path of the whole-row kernel (full-sort rows replayed over
// their distinct values): LDS for the row's patch table, a hash table of the
// distinct values and their sorted list.  Rows that need more take the
// whole-row sort.
constexpr int kGrpPatchCap = 2048;   // distinct patched ids (history window + bias)
constexpr int kGrpHashBits = 12;
constexpr int kGrpHashCap = 1 << kGrpHashBits;
constexpr int kGrpHashLimit = 3072;  // distinct values kept (load factor 3/4)
constexpr int64_t kGrpMaxV = 180224; // vocabularies whose bitmap fits beside the rest
inline size_t group_lds_bytes(int64_t V) {
  if (V < 1 || V > kGrpMaxV) return 0;
  const size_t nw = (size_t)((V + 31) / 32);
  return nw * 8 + (size_t)kGrpPatchCap * 16 + (size_t)kGrpHashCap * 16;
}

// The member search's dynamic LDS: the bitmap, its prefix counts and the
// patch table (the front of group_lds_bytes' layout).
inline size_t group_patch_lds_bytes(int64_t V) {
  if (V < 1 || V > kGrpMaxV) return 0;
  const size_t nw = (size_t)((V + 31) / 32);
  return nw * 8 + (size_t)kGrpPatchCap * 16;
}

struct GenericArgs {
  const float* logits;
  int64_t V;
  const RowParams* rp;
  const int32_t* hist;
  const int64_t* hist_len;
  int hcap;
  const int32_t* bias_ids;
  const float* bias_vals;
  const int32_t* generic_list;
  const int32_t* generic_count;  // this call's counter
  int32_t* next_count;           // the next call's counter, zeroed here
  // the next call's fallback and walk counts (fb_count, w_count below), which
  // every call zeroes whichever launches it makes (kept beside next_count: a
  // kernel that zeroes them reads no further kernel-argument line for them)
  int32_t* fb_next;
  int32_t* w_next;
  // the next unclaimed list position (workgroups claim rows one at a time;
  // null: workgroup w takes positions w, w + n, ...) and the next call's
  // claim counter, zeroed here
  int32_t* claim;
  int32_t* next_claim;
  uint32_t* scratch;             // per workgroup: 5 x vpad uint32
  int64_t vpad;
  const double* d_u;
  uint64_t* rng;
  int32_t* out;
  DebugPtrs dbg;
  int grouped;  // 1: the launch carries group_lds_bytes(V) of dynamic LDS
  const int32_t* row_done;  // [B] or null: a nonzero row samples nothing (out = -1)
  // rows known to need this path when the sampler was made (full sorts),
  // served before the listed ones; null: none
  const int32_t* fixed_list;
  int n_fixed;
  // Two launches (grouped rows first, then the rest): the first lists every
  // row it does not finish in fb_list (counted in fb_count), with the row's
  // uniform in fb_u when it drew it; the second takes that list (fb_in = 1)
  // as its list of rows.
  int32_t* fb_list;
  int32_t* fb_count;
  int list_cap;  // the batch: no list holds more rows (a push past it is dropped)
  double* fb_u;
  int fb_in;
  // The grouped rows' walks in a launch of their own (walk_split = 1): the
  // grouped launch stores each row's groups (gt_*, kGrpHashCap per row) and
  // lists the row in w_list; the walk launch walks them (one wave per row)
  // and, for a drawn value that occurs more than once, keeps the group's
  // count record and value key and the member's rank (p3_*) for its member
  // search.  Rows that fail any step go to the fallback list.
  int walk_split;
  float* gt_e;      // [B][kGrpHashCap] the groups' exponentials
  uint32_t* gt_c;   // [B][kGrpHashCap] their count records (count, or kGrpOne | index)
  uint32_t* gt_k;   // [B][kGrpHashCap] their value keys
  int32_t* gt_n;    // [B] the groups, | kGtComplete when they hold every candidate
  int32_t* w_list;
  int32_t* w_count;
  uint32_t* p3_rec;  // [B] the drawn group's count record
  uint32_t* p3_key;  // [B] its value key
  int64_t* p3_t;     // [B] the drawn member's rank among the group's members
};
// A row of the fallback list whose uniform the grouped launch drew (fb_u).
constexpr int32_t kFbUSaved = 1 << 30;
// gt_n: the groups hold every candidate of the row.
constexpr int32_t kGtComplete = 1 << 30;
// walk_member_kernel: rows walked side by side per workgroup, one wave each
constexpr int kWalkRows = 2;
// its dynamic LDS: the waves' walk tables (kGrpHashCap exponentials and
// counts each), later the member search's patch table
inline size_t walk_member_lds_bytes(int64_t V) {
  const size_t walk = (size_t)kWalkRows * kGrpHashCap * 8;
  const size_t search = group_patch_lds_bytes(V);
  return walk > search ? walk : search;
}

// floor_kernel: the full-sort rows of a batch of only such rows, each row
// split over slices of kFloorSlice values, one workgroup each.  A slice keeps
// its values within kGroupFloor of its maximum (at most kFloorKeep), and the
// last slice of a row to finish merges them (at most kFloorMerge) and runs the
// row's tail; any row it cannot finish goes to the whole-row list.
constexpr int kFloorThreads = 512;
constexpr int kFloorVec4 = 8;  // float4 per thread: the slice sits in registers
constexpr int kFloorSlice = kFloorThreads * kFloorVec4 * 4;
constexpr int kFloorPatchCap = 1024;  // patched ids per slice
constexpr int kFloorKeep = 2048;
constexpr int kFloorMerge = 2048;
constexpr int kFloorMaxSlices = 16;  // V <= 16 * kFloorSlice = 262144
// dynamic LDS: the slice's tables, then (reused) the merge's records and tail arrays
constexpr size_t kFloorLds1 = (size_t)kFloorSlice / 32 * 8 + (size_t)kFloorPatchCap * 16 + (size_t)kFloorKeep * 8;
constexpr size_t kFloorLds2 = (size_t)kFloorMerge * 20;
constexpr size_t kFloorLds = kFloorLds1 > kFloorLds2 ? kFloorLds1 : kFloorLds2;

struct FloorArgs {
  const float* logits;
  int64_t V;
  int B;
  int S;  // slices per row
  const RowParams* rp;
  const int32_t* hist;
  const int64_t* hist_len;
  int hcap;
  const int32_t* bias_ids;
  const float* bias_vals;
  int bstride;  // > 0: row b's bias list at b * bstride, padded with -1
  const double* d_u;
  uint64_t* rng;
  int32_t* out;
  DebugPtrs dbg;
  const int32_t* row_done;
  int32_t* generic_list;  // rows for the whole-row launch after this one
  int32_t* generic_count;
  uint64_t* part;      // [B][S][kFloorKeep] (key << 32 | index) of the kept values
  int32_t* part_n;     // [B][S] kept values, -1: the row goes to the whole-row launch
  uint32_t* part_max;  // [B][S] the slice maximum's key
  uint32_t* arrive;    // [B] slices finished (reset by the last)
};

struct StreamArgs {
  const float* logits;
  int64_t V;
  int B;
  int S;        // workgroups (slices) per row
  int L;        // slice length, a multiple of 4
  int xcd_map;  // 1: a row's slices are placed on one XCD (B % 8 == 0)
  const RowParams* rp;
  const int32_t* hist;
  const int64_t* hist_len;
  int hcap;
  const int32_t* bias_ids;
  const float* bias_vals;
  int bstride;  // > 0: row b's bias entries start at b * bstride
  // dynamic LDS layout: cand[2][ccap] u64 | region A
  int ccap;     // candidate buffer entries (each of two ping-pong buffers)
  int nwords;   // patch bitmap words, ceil(L / 32)
  int pcap;     // distinct patched ids per slice held in LDS
  int mcap;     // member sort capacity, a power of two >= 2k
  int kcap;     // >= every fast row's k
  int offA;     // byte offset of region A
  // slice exchange (S > 1)
  uint64_t* part_cand;  // [B*S*pc]
  SliceInfo* part_info; // [B*S]
  uint32_t* arrive;     // [B], zero between calls
  int pc;
  // outputs
  const double* d_u;
  uint64_t* rng;
  int32_t* out;
  int32_t* generic_list;
  int32_t* generic_count;  // this call's counter (zero on entry)
  DebugPtrs dbg;
  // gen_inline: rows handed on are served by the last workgroup of this
  // kernel (counted in `done`, zero between calls) instead of a second launch
  int gen_inline;
  uint32_t* done;
  int hbits;    // k64_kernel: log2 of the patch hash table's slots
  const int32_t* row_done;  // [B] or null: a nonzero row samples nothing (out = -1)
  // k64_kernel: the streamed rows, one per workgroup (a batch whose other
  // rows go to the whole-row kernel from its fixed list); null: workgroup b
  // takes row b
  const int32_t* row_list;
  int n_list;
  GenericArgs ga;
};


// k64_kernel instances by the streamed rows they serve
constexpr int kK64RowsAny = 0;     // greedy and top-k rows
constexpr int kK64RowsTopK = 1;    // top-k rows only
constexpr int kK64RowsGreedy = 2;  // greedy rows only

struct LaunchPlan {
  int nt;        // streaming workgroup size: 256, 512 (k > 64, two per CU) or 1024
  bool k64;      // k64_kernel instead of stream_kernel (wave path, one workgroup per row)
  int k64_rows;  // the kinds of streamed rows: kK64RowsAny, kK64RowsTopK or kK64RowsGreedy
  bool wave;     // every top-k row has k <= kWaveTopK: per-wave candidate buffers
  int q;         // per-thread top-Q of the threshold refresh: 1, 2, 4 or 8
  bool vec4;     // 16-byte loads (V % 4 == 0 and aligned logits)
  size_t lds;    // dynamic LDS bytes of the streaming kernel
  int gen_blocks;
  size_t gen_lds;  // dynamic LDS bytes of the whole-row kernel (grouped path), 0 = none
  bool no_stream;  // no row is a streaming row: the whole-row kernel alone, over every row
  int floor_slices;  // > 0: floor_kernel over every row (no streamed rows), then the whole-row launch
  int walk_blocks;  // walk launch (walk_member_kernel): workgroups, kWalkRows rows each at a time
  size_t walk_lds;  // and their dynamic LDS (walk_member_lds_bytes)
};

hipError_t launch_sample(const StreamArgs& sa, const GenericArgs& ga, const FloorArgs& fa, const LaunchPlan& lp,
                         hipStream_t s, hipEvent_t ev_start, hipEvent_t ev_stop, hipEvent_t gev_start,
                         hipEvent_t gev_stop);
hipError_t launch_accept_host(const int32_t* d_ids, const int32_t* d_cnt, int B, int count,
                              int32_t* hist, int64_t* hist_len, int hcap, int row_only, hipStream_t s);
// one batched generation step after the sampling: rows not done finish on an
// end-of-generation id, else accept theirs
hipError_t launch_clear_counters(uint32_t* arrive, int B, uint32_t* done, int32_t* gcount, hipStream_t s);
hipError_t launch_generate_step(const int32_t* d_out, int B, int64_t V, const int32_t* eog, int n_eog,
                                int32_t* row_done, int32_t* hist, int64_t* hist_len, int hcap, hipStream_t s);
hipError_t launch_accept_device(const int32_t* d_ids, int B, int64_t V, int32_t* hist,
                                int64_t* hist_len, int hcap, hipStream_t s);
hipError_t launch_expf(const float* x, float* y, int64_t n, hipStream_t s);
// topTokens over `rows` rows of V logits: n results per row (stride n), n <= kTopMaxN or V <= kTopMaxN
constexpr int kTopThreads = 1024;
constexpr int kTopMaxN = 2048;   // largest number of results per row (sorted in LDS)
hipError_t launch_argmax(const float* logits, int rows, int64_t V, int32_t* out, hipStream_t s);
hipError_t launch_row_nll(const float* logits, int rows, int64_t V, const int32_t* targets, double* out,
                          hipStream_t s);
hipError_t launch_top_tokens(const float* logits, int rows, int64_t V, int n, int32_t* ids,
                             float* probs, hipStream_t s);
// softmaxInPlace over `rows` rows of V logits (out may be logits), and
// logProb's per-token term; V < 2^29
hipError_t launch_softmax_rows(const float* logits, int rows, int64_t V, float* out, hipStream_t s);
hipError_t launch_log_prob(const float* logits, int rows, int64_t V, const int32_t* targets, float* prob,
                           double* logp, hipStream_t s);
hipError_t set_kernel_attributes();
size_t max_dynamic_lds();

// The output projection (nls_lmhead.hip): one matmul(m.output, x, y, nb).
struct LmHeadCall {
  const void* w;      // rows x row_bytes GGUF bytes
  int type;           // GGML type code
  int64_t rows, cols, row_bytes;
  const float* x;     // [nb, cols]
  int nb;
  float* y;           // [nb, rows]
  bool use_act;       // the int8 activation path (model.nim:185)
  int8_t* act_qs;     // [nb * cols] workspace
  float* act_d;       // [nb * cols / block] workspace
  const float* lora_a;
  const float* lora_b;
  int lora_rank;
  float lora_scale;
  float* lora_tmp;    // [nb * rank] workspace
};
constexpr int kLmMaxIntBlocks = 1024;  // blocks per row the int8 path's LDS holds
int lm_act_block_len(int type);
bool lm_type_supported(int type);
hipError_t launch_lm_head(const LmHeadCall& c, hipStream_t s);

}  // namespace nls
