// Internal launch interface between the C-ABI layer (mf_abi.cpp) and the
// kernel translation units.  Arguments are validated by the caller; these
// functions only build grids and launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mf {

struct Record;

// Where a head workgroup reads candidate scores from.
enum class ScoreSource : int {
  kDotF32 = 0,       // fast dot of FP32 normalized hidden with the FP16 table
  kDotF16Hidden = 1, // the same with FP16 hidden (legacy restricted head)
  kLookup = 2,       // FP32 scores already computed by the MFMA projection
};

struct HeadArgs {
  const float* y;            // [rows, H] FP32 normalized hidden
  const uint16_t* hidden16;  // [rows, H] FP16 hidden (kDotF16Hidden)
  const uint16_t* emb;       // [V, H] FP16 table
  const float* scores;       // [rows, V] (kLookup)
  const float* row_norm;     // [rows] ||y_r|| upper bounds (kLookup)
  const float* tok_norm;     // [V] ||e_t|| upper bounds (kLookup)
  const uint32_t* row_state; // CSR mode when non-null
  const uint32_t* offsets;
  const uint32_t* tokens;
  const uint32_t* fixed_ids;    // fixed-width mode [rows, max_allowed]
  const uint32_t* fixed_counts; // [rows]
  const uint32_t* state_next;   // [nnz] or null
  const int32_t* next_table;    // [states, V] or null
  uint32_t* out_token;
  float* out_score;
  uint32_t* out_next;
  Record* records;     // [rows, max_chunks] multi-workgroup rows
  uint32_t* counters;  // [rows] arrival counters (zero between calls)
  uint32_t rows;
  uint32_t H;
  uint32_t V;
  uint32_t states;
  uint32_t nnz;        // length of tokens: lists ending past it are invalid
  uint32_t max_allowed;
  uint32_t chunk;      // candidates per block
  uint32_t max_chunks; // chunk slots per row in the grid; 0 = one workgroup per row
  float coef;          // fast-score bound: b = coef * A + slack (dot), or
  float coef2;         //   b = ||e|| * (coef * ||y|| + coef2) + slack (lookup)
  float slack;
  int order;           // 0 fma chain, 1 mul-add chain
  int lookup_unrestricted; // kLookup: unrestricted rows score the whole vocabulary
  // Planned mode (CSR rows): work items are (row, chunk) pairs numbered by
  // prefix[rows + 1]; workgroup b owns items [W*b/G, W*(b+1)/G) and starts
  // its row walk at start_row[b].  Null prefix: grid of rows x max_chunks.
  const uint32_t* prefix;
  const uint32_t* start_row;
};

// Work plan built by the norm kernel's last workgroup (CSR decode tail):
// chunks per row, their exclusive prefix, and each head workgroup's first row.
// Invalid rows (state >= S, empty list) get their outputs written here and no
// chunk; unrestricted rows get no chunk (the MFMA fallback owns them).
struct PlanArgs {
  const uint32_t* row_state;
  const uint32_t* offsets;
  uint32_t states;
  uint32_t nnz;
  uint32_t max_chunks;      // rows needing more chunks are invalid
  uint32_t chunk;
  uint32_t head_groups;     // G
  uint32_t* chunks_per_row; // [rows]
  uint32_t* prefix;         // [rows + 1]
  uint32_t* start_row;      // [G]
  uint32_t* counter;        // arrival counter (zero between calls)
  uint32_t* out_token;
  float* out_score;
  uint32_t* out_next;
};

constexpr uint32_t kHeadChunkMax = 1024;
constexpr uint32_t kHeadMaxRecords = 256;
constexpr uint32_t kHeadMaxHidden = 8192;

hipError_t launch_rms_norm(const void* input, bool half_input,
                           const void* weight, bool half_weight, void* output,
                           bool half_output, float* row_norm, uint32_t rows,
                           uint32_t hidden, float epsilon, hipStream_t stream);

// RMSNorm (or a plain copy when weight is null) of FP32 rows into y with row
// norms, plus the work plan.
hipError_t launch_norm_plan(const float* x, const float* weight, float* y,
                            float* row_norm, uint32_t rows, uint32_t hidden,
                            float epsilon, const PlanArgs& plan,
                            hipStream_t stream);

hipError_t launch_head(ScoreSource source, const HeadArgs& args,
                       uint32_t groups, hipStream_t stream);

hipError_t launch_linear_f16_simple(const uint16_t* input, const uint16_t* weight,
                                    uint16_t* output, uint32_t rows,
                                    uint32_t in_features, uint32_t out_features,
                                    hipStream_t stream);

hipError_t launch_greedy(const void* logits, bool half, uint32_t* tokens,
                         uint32_t rows, uint32_t vocab, hipStream_t stream);

hipError_t launch_restricted_greedy(const void* logits, bool half,
                                    const uint32_t* allowed,
                                    const uint32_t* counts, uint32_t* tokens,
                                    uint32_t rows, uint32_t vocab,
                                    uint32_t max_allowed, hipStream_t stream);

hipError_t launch_fill_zero(void* address, uint64_t bytes, hipStream_t stream);

// ---- MFMA projection (mf_mfma.hip) ----------------------------------------

struct ProjArgs {
  // A operand rows: FP32 normalized hidden y[rows] selected through row_index
  // (null: identity) and split on the fly into FP16 hi + lo parts, or FP16
  // input rows used as they are (a16).
  const float* y;
  const uint16_t* a16;
  const uint32_t* row_index;
  uint32_t m;          // number of A rows
  uint32_t rows;       // bound of row_index entries (out-of-range rows read as 0)
  const uint16_t* emb; // [V, H] B operand (row-major, token-major)
  uint32_t H;
  uint32_t V;
  // epilogues (any subset)
  float* out_f32;      // [m, V] FP32 scores
  uint16_t* out_f16;   // [m, V] FP16 rounded scores
  float* tok_norm;     // [V] ||e_t|| upper bounds, written by M-tile 0
};

hipError_t launch_projection(const ProjArgs& args, hipStream_t stream);

// Full-vocabulary head for unrestricted rows: projection with a windowed
// argmax epilogue, per-tile records and a last-arriver merge per row that
// rescores the window in the reference order.
struct FallbackArgs {
  const float* y;           // [rows, H] normalized hidden (all rows)
  const uint32_t* row_index;// [m] unrestricted rows (entries >= rows are skipped)
  uint32_t m;
  uint32_t rows;
  const float* row_norm;    // [rows]
  const uint16_t* emb;
  uint32_t H;
  uint32_t V;
  Record* records;          // [m, tiles]
  uint32_t* counters;       // [ceil(m / 32)]
  uint32_t* out_token;
  float* out_score;
  uint32_t* out_next;
  float coef;               // b = ||e|| * (coef * ||y|| + coef2) + slack
  float coef2;
  float slack;
  int order;
};

uint32_t fallback_tiles(uint32_t vocab);
hipError_t launch_fallback(const FallbackArgs& args, hipStream_t stream);

} // namespace mf
