// Internal launch interface between the C-ABI layer (mf_abi.cpp) and the
// kernel translation units.  Arguments are validated by the caller; these
// functions only build grids and launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mf {

struct Record;
struct RowMeta;
struct TileRecord;

// Where a decode-tail gather workgroup reads candidate scores from.
enum class ScoreSource : int {
  kDotF32 = 0,  // fast dot of FP32 normalized hidden with the FP16 table
  kMfma = 1,    // MFMA dot of the FP16 hi/lo split of the hidden (H % 32 == 0)
  kLookup = 2,  // FP32 scores already computed by the MFMA projection
};

// The fixed-width restricted head of the reference API
// (restricted_output_head_f16): one workgroup per row, FP16 hidden.
struct HeadArgs {
  const uint16_t* hidden16;     // [rows, H]
  const uint16_t* emb;          // [V, H]
  const uint32_t* fixed_ids;    // [rows, max_allowed]
  const uint32_t* fixed_counts; // [rows]
  uint32_t* out_token;
  float* out_score;
  uint32_t rows;
  uint32_t H;
  uint32_t V;
  uint32_t max_allowed;
  uint32_t chunk;      // candidates per block
  float coef;          // fast-score bound: b = coef * sum|y e| + slack
  float slack;
  int order;           // 0 fma chain, 1 mul-add chain
};

constexpr uint32_t kHeadChunkMax = 1024;
constexpr uint32_t kHeadMaxRecords = 256;
// decode tail: rows staged in LDS by the norm and finalize kernels
constexpr uint32_t kHeadMaxHidden = 8192;
// restricted_output_head: hidden rows up to this width are staged in LDS as
// FP32; wider ones are read from global memory
constexpr uint32_t kHeadLdsHidden = 16384;

hipError_t launch_rms_norm(const void* input, bool half_input,
                           const void* weight, bool half_weight, void* output,
                           bool half_output, float* row_norm, uint32_t rows,
                           uint32_t hidden, float epsilon, hipStream_t stream);

hipError_t launch_head(const HeadArgs& args, hipStream_t stream);

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
hipError_t launch_read_floor(const void* address, uint64_t bytes, uint32_t* sink,
                             hipStream_t stream);

// ---- decode tail (mf_tail.hip) ----------------------------------------------

constexpr uint32_t kGatherTileMax = 256;
constexpr uint32_t kPlanRowsMax = 1024;  // rows the gather plans in LDS
constexpr uint32_t kGatherWaveTile = 64;  // candidates per wave tile (MFMA gather)

struct TailNormArgs {
  uint32_t rows;
  const float* x;          // [rows, H]
  const float* weight;     // [H] or null (x already normalized)
  float epsilon;
  float* y;                // [rows, H] reference-order normalized hidden
  float* row_inv;          // [rows] the reference's 1 / sqrt(mean + eps) (1: no norm)
  // The fast scores use z = x * w (x without a weight): the normalized row
  // up to the positive per-row factor inv, which orders scores alike.
  float* row_norm;         // [rows] upper bound of ||z||
  float* row_slack;        // [rows] absolute error term of the row's bounds
  uint16_t* y_hi;          // [rows, H] FP16 split of z: hi = rne(z), lo = rne(z - hi) (or null)
  uint16_t* y_lo;
  float slack;             // absolute term of the fast score itself
  float slack_scaled;      // absolute term of the reference score, per unit of 1 / inv
  uint32_t chain;          // 0: y and row_inv come from the gather launch's chain waves
  const uint32_t* row_state;
  const uint32_t* offsets;
  uint32_t states;
  uint32_t nnz;
  uint32_t max_count;      // longer lists make the row invalid
  uint32_t V;
  uint32_t H;
  RowMeta* row_meta;       // [rows]
  uint32_t* fb_map;        // [rows] row -> unrestricted list index (reset here)
  uint32_t* out_token;
  float* out_score;
  uint32_t* out_next;
  // Sequence table: row r's state is row_state[row_sequence[r]] and its next
  // state goes to out_next[row_sequence[r]] (null: index r); indices >=
  // capacity make the row invalid.  hold: an empty list keeps the state.
  const uint32_t* row_sequence;
  uint32_t capacity;
  uint32_t hold;
  // The MFMA head's panel (fb_panel null: none).  Workgroup rows + j
  // normalizes row fb_rows[j] again (the same arithmetic, so the same bits)
  // and writes slot j: its FP16 split into the panel, its norm bound and its
  // row (kInvalidToken when fb_rows[j] >= rows).
  const uint32_t* fb_rows; // [fb_m]
  uint32_t fb_m;
  uint16_t* fb_panel;      // [panel_tiles(fb_m)] x panel_tile_bytes(H)
  uint32_t* fb_slot_row;   // [fb_m]
  float* fb_slot_norm;     // [fb_m]
  float* fb_slot_slack;    // [fb_m]
  // Range index of the table pass (range_index null: none): per 192-token
  // range g of the vocabulary and row r, range_index[g * rows + r] =
  // {lo, hi, record, 0}: the positions [lo, hi) of the row's ids in the
  // range (lo = hi = 0: none) and the range's record index among the row's
  // non-empty ranges; row_tiles[r] = the row's record count, with
  // kRangesUnused set when the list is not strictly ascending or holds an
  // id >= V (the norm kernel then writes the row's single record itself:
  // rescore the whole list, or the invalid row).  Walk workgroups of the
  // norm launch build it (mf_prep.hpp).
  const uint32_t* tokens;  // the state lists (range index only)
  uint4* range_index;      // [ranges, rows]
  uint32_t* row_tiles;     // [rows]
  uint32_t ranges;
  TileRecord* records;     // [rows, max_recs]
  uint32_t max_recs;
  // Dense index (dense_spans null: none).  Walk workgroup r of the norm
  // launch indexes row r when its list is restricted, at least dense_min
  // long, strictly ascending and below V: per 192-token range g,
  // dense_spans[(g * rows + r) * 2 + {0, 1}] = {m0, m1, m2, lo}, {m3, m4,
  // m5, cnt} (the range's ids as a 192-bit mask, the list position of its
  // first id, their count); dense_flag[r] = 1 (else 0).  A one-workgroup
  // kernel after the launch (dense_choose_kernel) gives the longest indexed
  // lists kRowDense in row_meta: as many as fill the room dense_fb
  // unrestricted rows leave in their panels, then whole panels while the
  // lists of the next panel hold at least dense_panel_ids ids.
  uint4* dense_spans;      // [ranges, rows, 2]
  uint32_t* dense_flag;    // [rows]
  uint32_t dense_min;
  uint32_t dense_fb;       // unrestricted rows of the call
  uint32_t dense_sort;     // power of two >= rows (the ranking's size)
  uint64_t dense_panel_ids;
};

// row_tiles flag: the row's ranges are not used (its one record comes from
// the norm kernel).
constexpr uint32_t kRangesUnused = 0x80000000u;

// Panel of the MFMA head: per tile of kPanelRows slots, the slots' FP16
// split [slot][hi | lo][H + kPanelPad] halves -- the head's LDS image of its
// A operand, so the head copies it with plain 1 KiB global-to-LDS bursts.
// The pad makes the row stride 2 (mod 4) 16-byte bank groups out of the 16
// that gfx950's 64 LDS banks form (H % 32 == 0): a ds_read_b128 serves 16
// lanes per cycle, lanes 0-3, 12-15, 20-23, 24-27 in one cycle and 4-11,
// 16-19, 28-31 in the next (the same for lanes 32-63), so A rows r_i read at
// one K offset by the lanes of columns 0-3, 12-15 (and, separately, 4-11)
// meet no bank conflict when their r_i differ mod 8 -- true for 16
// consecutive rows.
constexpr uint32_t kPanelRows = 32;
constexpr uint32_t kPanelPad = 16;
__host__ __device__ constexpr uint64_t panel_tile_bytes(uint64_t H) {
  return kPanelRows * 2u * (H + kPanelPad) * 2u;
}
__host__ __device__ constexpr uint32_t panel_tiles(uint32_t m) {
  return (m + kPanelRows - 1) / kPanelRows;
}
// Tokens per tile of the MFMA head (one window record per row and tile) and
// of the table pass (one workgroup step); the largest panel tile the
// LDS-resident variants stage.
constexpr uint32_t kHeadTileTokens = 192;
// Rows the table pass plans in LDS (one per thread of its workgroup).
constexpr uint32_t kPassRowsMax = 256;
// The one-kernel tail for short lists: candidates per workgroup (one part
// of a row's list), parts per row, the LDS a workgroup may take for x, the
// weight and the staged candidate rows, and the rows whose arrival counters
// the workspace keeps at its start.
constexpr uint32_t kShortListMax = 128;
constexpr uint32_t kShortPartsMax = 16;
constexpr uint32_t kShortLdsBytes = 156u * 1024u;
constexpr uint32_t kShortCountRows = 4096;
constexpr uint32_t kPanelLdsMaxBytes = 76u * 1024u;

struct GatherArgs {
  const float* y;          // [rows, H]
  const uint16_t* y_hi;    // [rows, H] FP16 split (MFMA)
  const uint16_t* y_lo;
  const uint16_t* emb;     // [V, H]
  const float* scores;     // [rows, V] (lookup)
  const float* row_norm;   // (lookup, MFMA) bound of ||z||
  const float* row_slack;  // (lookup, MFMA) the row's absolute error term
  const float* tok_norm;   // (lookup)
  const uint32_t* tokens;  // state lists
  const RowMeta* row_meta;
  TileRecord* records;     // [rows, max_tiles]
  uint32_t rows;
  uint32_t H;
  uint32_t V;
  uint32_t tile;           // candidates per tile (<= kGatherTileMax)
  uint32_t max_tiles;
  uint32_t groups;         // compute units for the planned mode (0 = grid mode)
  // Chain waves (MFMA gather, planned mode): the first chain_groups
  // workgroups normalize rows 0 .. chain_rows - 1 in the reference order into
  // y_out / inv_out while the others gather (the fast scores need only z).
  const float* x;
  const float* weight;
  float epsilon;
  float* y_out;
  float* inv_out;
  uint32_t chain_rows;
  float coef;              // dot: b = coef * sum|y e| + slack
  float coef2;             // lookup, MFMA: b = ||e|| (coef ||y|| + coef2) + slack
  float slack;
};

struct FinalizeArgs {
  const float* y;
  // records scored on z = x * w (row_inv given) or on y (null); exact
  // scores tighten a window only after conversion to the records' scale
  const float* row_inv;
  const uint16_t* emb;
  const uint32_t* tokens;
  const RowMeta* row_meta;
  const TileRecord* records;     // gather tiles [rows, max_tiles]
  uint32_t max_tiles;
  uint32_t tile;
  const TileRecord* fb_records;  // MFMA tiles [m, fb_tiles] (or null)
  const uint32_t* fb_map;
  uint32_t fb_tiles;
  int lookup_unrestricted;       // unrestricted rows live in records (comparator)
  const uint32_t* state_next;
  const int32_t* next_table;
  uint32_t* out_token;
  float* out_score;
  uint32_t* out_next;
  const uint32_t* row_sequence;  // as in TailNormArgs
  uint32_t capacity;
  // records per restricted row: row_tiles[r] & ~kRangesUnused (table pass),
  // or one per `tile` candidates of the list (null)
  const uint32_t* row_tiles;
  uint32_t rows;
  uint32_t H;
  uint32_t V;
  int order;
};

// Where row r's next state goes: out_next[row_sequence[r]] with a sequence
// table, else out_next[r]; null when there is no output or the index is
// outside the table.
__device__ __forceinline__ uint32_t* next_state_slot(uint32_t* out_next,
                                                     const uint32_t* row_sequence,
                                                     uint32_t capacity, uint32_t r) {
  if (out_next == nullptr) return nullptr;
  const uint32_t q = row_sequence != nullptr ? row_sequence[r] : r;
  return q < capacity ? out_next + q : nullptr;
}

hipError_t launch_tail_norm(const TailNormArgs& args, hipStream_t stream);
hipError_t launch_gather(ScoreSource source, const GatherArgs& args, hipStream_t stream);
hipError_t launch_gather_mfma(const GatherArgs& args, hipStream_t stream);  // mf_gather.hip
hipError_t launch_finalize(const FinalizeArgs& args, hipStream_t stream);

// ---- MFMA projection (mf_gemm.hip) ----------------------------------------

struct ProjArgs {
  const uint16_t* a16; // [m, H] FP16 A operand rows
  uint32_t m;          // number of A rows
  const uint16_t* emb; // [V, H] B operand (row-major, token-major)
  uint32_t H;          // a multiple of 32; rows 16-byte aligned
  uint32_t V;
  // exactly one of the two outputs
  float* out_f32;      // [m, V] FP32 scores
  uint16_t* out_f16;   // [m, V] FP16 rounded scores
  float* tok_norm;     // [V] ||e_t|| upper bounds, written by M-tile 0 (or null)
};

hipError_t launch_projection(const ProjArgs& args, hipStream_t stream);

// Full-vocabulary head for unrestricted rows: projection with a windowed
// argmax epilogue, per-tile records and a last-arriver merge per row that
// rescores the window in the reference order.
struct FallbackArgs {
  const uint16_t* panel;    // the norm kernel's panel of the m unrestricted rows
  const uint32_t* slot_row; // [m] source row of each slot (kInvalidToken: none)
  const float* slot_norm;   // [m] bound of ||z|| of each slot's row
  const float* slot_slack;  // [m] absolute error term of each slot's row
  uint32_t m;
  const uint16_t* emb;
  uint32_t H;
  uint32_t V;
  TileRecord* records;      // [m, tiles] (fallback_tiles(V) tiles of 192 tokens)
  uint32_t* fb_map;         // [rows] written: row -> slot
  uint32_t groups;          // compute units: workgroups per M-tile
  uint32_t tiles_per_group; // set by the launcher
  float coef;               // b = ||e|| * (coef * ||z|| + coef2) + slot slack
  float coef2;
};

uint32_t fallback_tiles(uint32_t vocab);
hipError_t launch_fallback(const FallbackArgs& args, hipStream_t stream);

// ---- table pass (mf_pass.hip) ------------------------------------------------
//
// One launch over the table in 192-token tiles serves the unrestricted rows
// (the head above, its records and fb_map) and the restricted candidates
// whose ids fall in each tile (the range index of the norm kernel), which
// get one window record per (row, tile) in `records`.
struct PassArgs {
  FallbackArgs head;          // m = 0: no unrestricted rows
  const RowMeta* row_meta;
  const uint32_t* row_tiles;  // [rows]
  const uint4* range_index;   // [ranges, rows] {lo, hi, record, 0}
  const uint32_t* tokens;     // state lists
  const uint16_t* z_hi;       // [rows, H] FP16 hi of z = x * w
  const float* row_norm;      // [rows] bound of ||z||
  const float* row_slack;     // [rows]
  TileRecord* records;        // [rows, max_recs]
  uint32_t max_recs;
  uint32_t rows;
  uint32_t ranges;
  float coef;                 // candidate bound: b = ||e|| (coef ||z|| + coef2) + slack
  float coef2;
};

hipError_t launch_pass(const PassArgs& args, hipStream_t stream);

// ---- dense head (mf_dense.hip) -------------------------------------------------
//
// One launch over the table in 192-token tiles for the unrestricted rows
// (fb_rows) and the kRowDense rows: slot j < fb_m is fb_rows[j] (when that is
// an unrestricted row), then the kRowDense rows in row order; slot j's record
// of tile t is records[j * ranges + t] (the MFMA head's format; list
// positions for kRowDense rows), and fb_map[row] = j.
constexpr uint32_t kDensePanelSlots = 256;
struct DenseArgs {
  const uint16_t* emb;        // [V, H]
  const uint16_t* z_hi;       // [rows, H] FP16 hi of z = x * w
  const float* row_norm;      // [rows]
  const float* row_slack;     // [rows]
  const RowMeta* row_meta;    // kinds after the norm launch
  const uint4* spans;         // the norm launch's dense index
  const uint32_t* fb_rows;    // [fb_m]
  uint32_t fb_m;
  uint32_t rows;
  uint32_t H;
  uint32_t V;
  uint32_t ranges;            // 192-token tiles of the vocabulary
  TileRecord* records;        // [fb_m + rows, ranges]
  uint32_t* fb_map;           // [rows]
  float coef;                 // b = ||e|| (coef ||z|| + coef2) + slack (FP16 hi of z)
  float coef2;
  uint32_t groups;            // workgroups: compute units, a multiple of 8 (XCDs)
};
// Slots one launch serves: (groups / 8) panels of kDensePanelSlots.
hipError_t launch_dense(const DenseArgs& args, hipStream_t stream);
// mf_short.hip: candidate rows one workgroup can stage (0: H does not
// fit), and the one-kernel tail.  A row's list is cut into parts of
// per_part candidates, one workgroup each; when a row has several, each
// part leaves its selection in records[row * parts + part] and the last to
// arrive on counts[row] (zero between calls: that part sets it back) merges
// them.
struct ShortPartRecord {
  float score;
  uint32_t token;
  uint32_t pos;
  uint32_t next;       // next state of the best candidate
  uint32_t min_token;  // lowest id (an all-NaN row's selection)
  uint32_t min_pos;
  uint32_t min_next;
  uint32_t invalid;
};
struct ShortSplit {
  ShortPartRecord* records;  // [rows, parts]
  uint32_t* counts;          // [rows]
  uint32_t per_part;         // <= short_stage_rows(H, ...)
  uint32_t parts;            // ceil(max_count / per_part) <= kShortPartsMax
};
uint32_t short_stage_rows(uint32_t H, uint32_t max_count);
hipError_t launch_short(const TailNormArgs& norm, const FinalizeArgs& fin, const ShortSplit& split,
                        hipStream_t stream);

} // namespace mf
