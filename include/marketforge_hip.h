/*
 * marketforge_hip.h -- C ABI of the MI355X (gfx950) restricted output head.
 *
 * This is the drop-in boundary for the reference's CUDA operator layer
 * (the headers include/marketforge/cuda/greedy.hpp, rms_norm.hpp, linear.hpp).  Every entry point takes plain device
 * addresses (uintptr_t) with their allocation sizes in bytes -- the
 * (DeviceAddress, size_bytes) pair of the reference DeviceBuffer
 * (include/marketforge/cuda/device_buffer.hpp:20-56) -- and a stream handle
 * (StreamHandle, include/marketforge/cuda/cuda_stream.hpp:10-17).  No vendor
 * or torch type appears here.
 *
 * Conventions kept from the reference:
 *   - ops borrow caller buffers: they never allocate and never
 *     synchronize;
 *   - work is asynchronous on the caller's stream;
 *   - validation happens before any launch, in the reference order: zero
 *     dimensions / bad epsilon / null stream -> MF_INVALID_ARGUMENT; limits ->
 *     MF_RESOURCE_LIMIT; overflow -> MF_ARITHMETIC_OVERFLOW; mismatched sizes
 *     or aliased buffers -> MF_INVALID_ARGUMENT;
 *   - launch errors -> MF_DEVICE_BACKEND_FAILURE, runtime errors ->
 *     MF_DEVICE_RUNTIME_FAILURE, with the native HIP error code as detail
 *     (the reference's cuda_backend_failure / cuda_runtime_failure,
 *     src/cuda/cuda_internal.hpp:21-35);
 *   - a row that is invalid on the device produces MF_INVALID_TOKEN, not an
 *     error (src/cuda/greedy.cu:147-149, 163-166, 206-211).
 *
 * Selection rule everywhere (src/cuda/greedy.cu:84-100, 177-211): the winner
 * is the lowest token id among the maximal non-NaN scores (-0 == +0 tie); a
 * candidate set whose scores are all NaN selects its lowest id.
 */
#ifndef MARKETFORGE_HIP_H
#define MARKETFORGE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MF_ABI_VERSION 6u

/* Status: include/marketforge/core/status.hpp:7-49.  The numeric codes equal
 * the reference ErrorCode enumerators so results stay schema-compatible. */
typedef struct mf_status {
  int32_t code;
  uint32_t detail;
} mf_status;

enum mf_error_code {
  MF_OK = 0,
  MF_INVALID_ARGUMENT = 1,
  MF_UNSUPPORTED_DTYPE = 2,
  MF_INVALID_SHAPE = 3,
  MF_ARITHMETIC_OVERFLOW = 5,
  MF_ALLOCATION_FAILED = 7,
  MF_RESOURCE_LIMIT = 15,
  MF_DEVICE_BACKEND_FAILURE = 21, /* reference: cuda_backend_failure */
  MF_DEVICE_RUNTIME_FAILURE = 22  /* reference: cuda_runtime_failure */
};

/* include/marketforge/cuda/greedy.hpp:11-12 */
#define MF_INVALID_TOKEN 0xFFFFFFFFu
/* Row states of the decode tail (no reference counterpart: the
 * packed decode tail).  A state below the table's state count restricts the row to
 * that state's list; MF_STATE_UNRESTRICTED scores the whole vocabulary (the
 * MFMA fallback); any other value makes the row invalid. */
#define MF_STATE_UNRESTRICTED 0xFFFFFFFEu
#define MF_STATE_INVALID 0xFFFFFFFFu

/* Reference summation orders for one score (both FP32, FP16 table widened):
 *   MF_ORDER_FMA_CHAIN      s = fmaf(h[f], e[f], s), f = 0..H-1
 *                           (src/cuda/greedy.cu:171-176,
 *                            tests/cuda/cuda_tests.cu:739-744)
 *   MF_ORDER_MUL_ADD_CHAIN  s = s + h[f] * e[f] (two roundings), f = 0..H-1
 *                           (src/cpu/operators.cpp:584-595, linear_f32)
 * Chosen tokens and reported scores are bit-identical to that order. */
enum mf_dot_order { MF_ORDER_FMA_CHAIN = 0, MF_ORDER_MUL_ADD_CHAIN = 1 };

/* A device allocation: address and size in bytes (a DeviceBuffer view). */
typedef struct mf_buffer {
  uintptr_t address;
  uint64_t bytes;
} mf_buffer;

uint32_t mf_abi_version(void);
mf_status mf_device_count(int32_t* count);

/* ---- device plumbing ---------------------------------------------------- */

/* DeviceBuffer::allocate, src/cuda/device_buffer.cu:36-55 (0 bytes -> 0). */
mf_status mf_device_alloc(uint64_t bytes, uintptr_t* address);
/* DeviceBuffer::release, src/cuda/device_buffer.cu:105-114. */
mf_status mf_device_free(uintptr_t address);
/* DeviceBuffer::copy_from_host_async, src/cuda/device_buffer.cu:71-86. */
mf_status mf_copy_to_device_async(mf_buffer destination, uint64_t offset,
                                  const void* source, uint64_t bytes,
                                  uintptr_t stream);
/* DeviceBuffer::copy_to_host_async, src/cuda/device_buffer.cu:88-103. */
mf_status mf_copy_to_host_async(void* destination, mf_buffer source,
                                uint64_t offset, uint64_t bytes,
                                uintptr_t stream);
/* CudaStream::create (non-blocking), src/cuda/cuda_stream.cu:11-20. */
mf_status mf_stream_create(uintptr_t* stream);
/* CudaStream::release, src/cuda/cuda_stream.cu:39-47. */
mf_status mf_stream_destroy(uintptr_t stream);
/* CudaStream::synchronize, src/cuda/cuda_stream.cu:31-37. */
mf_status mf_stream_synchronize(uintptr_t stream);

/* ---- reference operators ------------------------------------------------ */

/* rms_norm_f32, include/marketforge/cuda/rms_norm.hpp:18-22.  Bit-identical
 * to the reference FP32 CPU order (src/cpu/operators.cpp:523-535); input and
 * output may alias, weight may not. */
mf_status mf_rms_norm_f32(mf_buffer input, mf_buffer weight, mf_buffer output,
                          uint64_t rows, uint64_t hidden_size, float epsilon,
                          uintptr_t stream);
/* rms_norm_f16, include/marketforge/cuda/rms_norm.hpp:24-28: the same FP32
 * arithmetic on decoded halves, output rounded to nearest even. */
mf_status mf_rms_norm_f16(mf_buffer input, mf_buffer weight, mf_buffer output,
                          uint64_t rows, uint64_t hidden_size, float epsilon,
                          uintptr_t stream);

/* greedy_select_f16, include/marketforge/cuda/greedy.hpp:17-21. */
mf_status mf_greedy_select_f16(mf_buffer logits, mf_buffer token_ids,
                               uint64_t rows, uint64_t vocabulary_size,
                               uintptr_t stream);
/* FP32-logit variant of greedy_select_f16 (same rules on binary32 values). */
mf_status mf_greedy_select_f32(mf_buffer logits, mf_buffer token_ids,
                               uint64_t rows, uint64_t vocabulary_size,
                               uintptr_t stream);

/* restricted_greedy_select_f16, include/marketforge/cuda/greedy.hpp:29-33. */
mf_status mf_restricted_greedy_select_f16(mf_buffer logits,
                                          mf_buffer allowed_token_ids,
                                          mf_buffer allowed_token_counts,
                                          mf_buffer token_ids, uint64_t rows,
                                          uint64_t vocabulary_size,
                                          uint64_t maximum_allowed_tokens,
                                          uintptr_t stream);
/* FP32-logit variant of restricted_greedy_select_f16. */
mf_status mf_restricted_greedy_select_f32(mf_buffer logits,
                                          mf_buffer allowed_token_ids,
                                          mf_buffer allowed_token_counts,
                                          mf_buffer token_ids, uint64_t rows,
                                          uint64_t vocabulary_size,
                                          uint64_t maximum_allowed_tokens,
                                          uintptr_t stream);

/* restricted_output_head_f16, include/marketforge/cuda/greedy.hpp:43-49.
 * Tokens are bit-identical to the reference kernel's sequential fmaf chain
 * (src/cuda/greedy.cu:133-212). */
mf_status mf_restricted_output_head_f16(mf_buffer hidden, mf_buffer embedding,
                                        mf_buffer allowed_token_ids,
                                        mf_buffer allowed_token_counts,
                                        mf_buffer token_ids, uint64_t rows,
                                        uint64_t hidden_size,
                                        uint64_t vocabulary_size,
                                        uint64_t maximum_allowed_tokens,
                                        uintptr_t stream);

/* linear_f16, include/marketforge/cuda/linear.hpp:18-22 (the reference's
 * cuBLAS GemmEx call, src/cuda/linear.cu:92-102): FP16 in, FP32 MFMA
 * accumulation, FP16 out.  No BLAS handle: the GEMM is this library's own
 * MFMA kernel. */
mf_status mf_linear_f16(mf_buffer input, mf_buffer weight, mf_buffer output,
                        uint64_t rows, uint64_t input_features,
                        uint64_t output_features, uintptr_t stream);

/* ---- the packed decode tail (no single reference call) ------------------ */
/* Per row r: y = RMSNorm(x[r]) (operators.cpp:523-535 order); score the
 * allowed ids of row_state[r] against the FP16 tied embedding in the chosen
 * reference order; select (greedy.cu rules); advance the DFA.  Restricted
 * rows gather their CSR list on the device; rows listed in unrestricted_rows
 * (row_state == MF_STATE_UNRESTRICTED) go to the MFMA full-vocabulary head.
 *
 * State table (device-resident, built once): state_offsets u32[states + 1],
 * state_tokens u32[nnz] with distinct ids per state (the TokenDfa arcs,
 * src/grammar/token_dfa.cpp:100-109).  DFA advance uses either
 * state_next u32[nnz] (arc next states, token_dfa.cpp:111-128: the next state
 * of the chosen arc) or next_table i32[states, vocab] (-1 = disallowed; the
 * u32 view of the looked-up value is stored).  Both absent: no advance.
 *
 * Outputs: out_token u32[rows]; out_score f32[rows] (the chosen token's score
 * in the chosen order, NaN for invalid rows; optional); out_next_state
 * u32[rows] (optional; MF_STATE_INVALID for invalid rows,
 * MF_STATE_UNRESTRICTED for unrestricted rows).
 *
 * Sequence table (row_sequence given, for continuous batching): row_state is
 * then a table of per-sequence DFA states with capacity = row_state.bytes / 4
 * entries.  Row r reads its state at row_state[row_sequence[r]] and writes its
 * next state to out_next_state[row_sequence[r]]; out_next_state has the
 * table's size and may be row_state itself (the table is updated in place).
 * A row whose index is >= capacity is invalid and writes no state.  The
 * sequences of one call must be distinct: two rows with one index race.
 *
 * flags: MF_TAIL_HOLD_FINISHED -- a row whose state has an empty list (a
 * terminal state of the token DFA: its trie ends every choice at a leaf and
 * extends no choice through one, src/grammar/token_dfa.cpp:49-53, 67-71) writes its own state as next state
 * (token MF_INVALID_TOKEN, score NaN), so a decode loop can run past a
 * sequence's end with no host check.  Without the flag such a row's next
 * state is MF_STATE_INVALID, as for every invalid row.
 *
 * flags: MF_TAIL_SORTED_LISTS -- every state's list is strictly ascending,
 * as TokenDfa keeps its arcs (src/grammar/token_dfa.cpp:100-109).  When the
 * call has unrestricted rows (so the whole table is read anyway), or with
 * MF_TAIL_TABLE_PASS as well, and hidden % 64 == 0, hidden <= 576 and
 * rows <= 256, the tail then scores the restricted and the unrestricted
 * rows in one pass over the table (the restricted-stage entry point runs
 * it; the unrestricted one does nothing).  Results are the same with or
 * without the flags; a list that turns out not to be ascending is rescored
 * in full, exactly.  MF_TAIL_TABLE_PASS alone changes nothing.
 *
 * Dense head: otherwise, with MF_TAIL_SORTED_LISTS, hidden % 32 == 0,
 * hidden >= 1024, rows <= 8191, vocab < 2^19 (the device's ranking packs
 * (count, row) into 32 bits) and rows + unrestricted_count within the
 * launch's panels (256 slots per 8 compute units: 8192 on MI355X), the
 * unrestricted stage
 * runs one pass over the table that scores the unrestricted rows and the
 * long ascending lists (at least vocab / 256 and 64 ids) with MFMA against
 * every token, keeping only the allowed ones; the gather skips those rows.
 * The device takes the longest lists, as many as fill the room the
 * unrestricted rows leave in their panels of 256 slots, then whole panels
 * while the lists of the next panel hold at least 5/2 vocab ids (a panel's
 * pass costs about as much as gathering that many rows).
 * MF_TAIL_NO_DENSE keeps every restricted row on the gather.  The results
 * are the same.
 *
 * Short lists: a call with no unrestricted rows, hidden % 8 == 0 and every
 * list within 16 parts of one workgroup's LDS stage of candidate rows (128
 * at hidden <= 576) runs as ONE kernel in the prepare stage (norm, exact
 * reference-order scores of every candidate, selection and DFA advance; the
 * other three stages do nothing), unless the table pass is chosen above or
 * flags hold MF_TAIL_NO_FUSED.  When a list takes more than one part, the
 * pack must also fit rows x parts <= 512 workgroups and rows <= 4096; the
 * last part of a row to finish merges the parts.  The results are the same.
 *
 * Workspace: caller-allocated device memory of mf_decode_tail_workspace_bytes
 * bytes, zero-filled once by mf_workspace_init before first use.  It starts
 * with the one-kernel tail's per-row arrival counters, which every call of
 * any shape leaves at zero; the rest is scratch.  Every call leaves it ready
 * for the next one; calls that overlap in time on the same workspace race. */
typedef struct mf_decode_tail_args {
  mf_buffer x;                 /* f32 [rows, hidden] (pre-norm hidden) */
  mf_buffer norm_weight;       /* f32 [hidden]; address 0: x is already normalized */
  float epsilon;
  int32_t order;               /* enum mf_dot_order */
  mf_buffer embedding;         /* f16 [vocab, hidden] */
  mf_buffer row_state;         /* u32 [rows] */
  mf_buffer state_offsets;     /* u32 [states + 1] */
  mf_buffer state_tokens;      /* u32 [nnz] */
  mf_buffer state_next;        /* u32 [nnz] or address 0 */
  mf_buffer next_table;        /* i32 [states, vocab] or address 0 */
  mf_buffer unrestricted_rows; /* u32 [unrestricted_count] or address 0 */
  mf_buffer out_token;         /* u32 [rows] */
  mf_buffer out_score;         /* f32 [rows] or address 0 */
  mf_buffer out_next_state;    /* u32 [rows] or address 0 */
  mf_buffer workspace;
  uint64_t rows;
  uint64_t hidden;
  uint64_t vocab;
  uint64_t states;
  uint64_t nnz;
  uint64_t max_count;          /* longest state list (table builder's figure) */
  uint64_t unrestricted_count;
  mf_buffer row_sequence;      /* u32 [rows] or address 0: see "Sequence table" */
  uint64_t flags;              /* MF_TAIL_HOLD_FINISHED | MF_TAIL_SORTED_LISTS | MF_TAIL_TABLE_PASS
                                  | MF_TAIL_NO_FUSED | MF_TAIL_NO_DENSE */
} mf_decode_tail_args;

#define MF_TAIL_HOLD_FINISHED 1u
#define MF_TAIL_SORTED_LISTS 2u
#define MF_TAIL_TABLE_PASS 4u
#define MF_TAIL_NO_FUSED 8u
#define MF_TAIL_NO_DENSE 16u

mf_status mf_decode_tail_workspace_bytes(const mf_decode_tail_args* args,
                                         uint64_t* bytes);

/* Which kernels mf_decode_tail_f16 runs for these arguments (no reference
 * counterpart; for benchmarks and tests that report per-kernel figures):
 * MF_TAIL_PATH_GATHER (restricted stage = CSR gather, unrestricted stage =
 * MFMA head) or MF_TAIL_PATH_TABLE_PASS (restricted stage = one pass over
 * the table for both kinds of rows, unrestricted stage empty) or
 * MF_TAIL_PATH_FUSED (the whole tail in the prepare stage's one kernel) or
 * MF_TAIL_PATH_DENSE (restricted stage = CSR gather of the rows the dense
 * head leaves, unrestricted stage = the dense head). */
#define MF_TAIL_PATH_GATHER 0u
#define MF_TAIL_PATH_TABLE_PASS 1u
#define MF_TAIL_PATH_FUSED 2u
#define MF_TAIL_PATH_DENSE 3u
mf_status mf_decode_tail_path(const mf_decode_tail_args* args, uint32_t* path);
/* Zero-fills a workspace with a fill kernel (safe under graph capture). */
mf_status mf_workspace_init(mf_buffer workspace, uintptr_t stream);
/* Reads every byte of `data` once (16-byte loads, whole 16-byte words; the
 * address 16-byte aligned) and writes nothing but, in practice never, one
 * word of `sink`.  No counterpart in the reference: the read-bandwidth floor
 * a benchmark times next to a kernel that streams the same bytes (e.g. the
 * table pass over the embedding). */
mf_status mf_read_floor(mf_buffer data, mf_buffer sink, uintptr_t stream);

/* The restricted path: CSR gather for restricted rows + MFMA fallback.
 * Equivalent to the four stages below, in order, on one stream. */
mf_status mf_decode_tail_f16(const mf_decode_tail_args* args, uintptr_t stream);

/* mf_decode_tail_f16 without a caller workspace and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The workspace is a device array inside
 * the library, mf_decode_tail_noalloc_max_bytes() bytes (16 MiB) per GPU,
 * held from library load until the process ends; args->workspace is not
 * used.  Same kernels, same results as mf_decode_tail_f16.  A call whose
 * workspace (mf_decode_tail_workspace_bytes) exceeds the array returns
 * MF_RESOURCE_LIMIT before any launch.  The first successful call on a
 * device looks up that device's array and zero-fills it on the call's stream
 * (a fill kernel, no memset node); until then every call tries again, and a
 * first call on a stream under graph capture returns
 * MF_DEVICE_RUNTIME_FAILURE with detail hipErrorStreamCaptureUnsupported
 * before any launch, so make one eager call on each device before capturing.
 * Every call on one GPU shares that GPU's array: calls that overlap in time
 * on one GPU (two streams, two threads) race and must be ordered by the
 * caller. */
uint64_t mf_decode_tail_noalloc_max_bytes(void);
mf_status mf_decode_tail_f16_noalloc(const mf_decode_tail_args* args, uintptr_t stream);

/* Stages of mf_decode_tail_f16 for callers that schedule them separately
 * (e.g. the unrestricted stage on a second stream once prepare is done).
 * prepare:      final RMSNorm into the workspace, per-row metadata, the FP16
 *               split of unrestricted rows; presets invalid rows' outputs.
 * restricted:   CSR gather of the restricted rows into tile records (table
 *               pass: both kinds of rows, see MF_TAIL_SORTED_LISTS).
 * unrestricted: MFMA full-vocabulary head of unrestricted_rows into tile
 *               records (table pass: nothing).
 * finalize:     per row, merges the records, rescores the surviving
 *               candidates in the reference order, writes the outputs.
 * restricted and unrestricted need prepare; finalize needs both. */
mf_status mf_decode_tail_prepare(const mf_decode_tail_args* args, uintptr_t stream);
mf_status mf_decode_tail_restricted(const mf_decode_tail_args* args, uintptr_t stream);
mf_status mf_decode_tail_unrestricted(const mf_decode_tail_args* args,
                                      uintptr_t stream);
mf_status mf_decode_tail_finalize(const mf_decode_tail_args* args, uintptr_t stream);

/* The full-output-projection comparator for the same contract: a GEMM
 * projection of every row over the whole vocabulary into FP32 scores (the
 * library's own MFMA projection kernel, the normalized row split into FP16
 * hi and lo parts, FP32 accumulation), then the restricted selection over
 * those scores (the shape of the reference's "full" path,
 * src/tools/cuda_restricted_output_head_bench.cu:181-191).  Outputs are
 * bit-identical to mf_decode_tail_f16.  Needs
 * mf_decode_tail_full_workspace_bytes of workspace. */
mf_status mf_decode_tail_full_workspace_bytes(const mf_decode_tail_args* args,
                                              uint64_t* bytes);
mf_status mf_decode_tail_full_f16(const mf_decode_tail_args* args,
                                  uintptr_t stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* MARKETFORGE_HIP_H */
