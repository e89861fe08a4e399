/*
 * CPU oracle for the restricted output head hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.  The
 * product path (market_sim_amd) never calls it and has no CPU fallback.
 *
 * Each function restates one reference loop in the same operation order, so
 * that results are bit-identical to the reference's FP32 CPU arithmetic.  The
 * file must be compiled with -ffp-contract=off and without fast-math (see
 * oracle/Makefile): every `a * b + c` below is two roundings unless it is an
 * explicit fmaf().
 *
 * Pinning (how each function is checked; details in tests/test_oracle_*.py):
 *   orc_half_to_float / orc_float_to_half  numpy float16 casts (IEEE RNE),
 *                                          every one of the 65536 halves.
 *   orc_rms_norm_f32     reference operators.cpp compiled into oracle/_ref,
 *                        bit-exact; hand values of cpu_operator_tests.cpp:59-108.
 *   orc_rms_norm_f16     numpy's IEEE float32 -> float16 cast of the reference
 *                        rms_norm_f32 (oracle/_ref) on the decoded inputs, bit
 *                        for bit, with half-subnormal and overflowing outputs;
 *                        x * (inv * w) and a pairwise sum of squares shown to
 *                        differ (tests/test_oracle_pin_f16_norm_f32_table.py).
 *   orc_dot_fma          the ascending single-rounding chain evaluated in
 *                        exact rational arithmetic on rows spanning many
 *                        binades, bit for bit (tests/test_oracle_fma_pin.py,
 *                        which also shows that reversed, unfused, strided and
 *                        pairwise chains differ on those rows); tiny head
 *                        known answer (cuda_tests.cu:699-800): tokens
 *                        [14, 8, 1] and exact rational scores.
 *   orc_dot_mul_add      reference linear_f32 in oracle/_ref, bit-exact;
 *                        linear known answer [-2, 3].
 *   dot_in_order_f32     (FP32 table, both orders) exact rational chains on
 *                        rows spanning many binades, reached through
 *                        orc_decode_tail with one candidate per row; other
 *                        orders shown to differ on the same rows
 *                        (tests/test_oracle_pin_f16_norm_f32_table.py).
 *   orc_select_*         greedy/restricted tie, NaN and sentinel cases of
 *                        cuda_tests.cu:508-565, 567-697, 1173-1277, 1341-1403;
 *                        real SmolLM2 logits fixture -> [198, 198, 504].
 *   orc_decode_tail      brute-force argmax in float64 with margin qualification,
 *                        one-hot closed forms, full-vocab == restricted(all ids).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_INVALID_TOKEN 0xFFFFFFFFu
#define ORC_STATE_UNRESTRICTED 0xFFFFFFFEu
#define ORC_ORDER_FMA_CHAIN 0
#define ORC_ORDER_MUL_ADD_CHAIN 1

/* ------------------------------------------------------------------------ */
/* IEEE binary16 <-> binary32                                                */
/* ------------------------------------------------------------------------ */

float orc_half_to_float(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t exponent = ((uint32_t)h >> 10) & 0x1fu;
  const uint32_t mantissa = (uint32_t)h & 0x3ffu;
  uint32_t bits;
  float value;
  if (exponent == 0) {
    /* zero or subnormal: mantissa * 2^-24, exact in binary32 */
    value = (float)mantissa * 0x1p-24f;
    memcpy(&bits, &value, 4);
    bits |= sign;
  } else if (exponent == 31) {
    bits = sign | 0x7f800000u | (mantissa << 13);
  } else {
    bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
  }
  memcpy(&value, &bits, 4);
  return value;
}

/* Round-to-nearest-even binary32 -> binary16 (the __float2half_rn rule). */
uint16_t orc_float_to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) {
    if (ax > 0x7f800000u) {
      return (uint16_t)(sign | 0x7e00u); /* quiet NaN */
    }
    return (uint16_t)(sign | 0x7c00u);
  }
  const int exponent = (int)(ax >> 23) - 127;
  const uint32_t mantissa = ax & 0x7fffffu;
  if (exponent >= -14) {
    /* normal half (or overflow after rounding) */
    if (exponent > 15) {
      return (uint16_t)(sign | 0x7c00u);
    }
    uint32_t base = ((uint32_t)(exponent + 15) << 10) | (mantissa >> 13);
    const uint32_t rest = mantissa & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (base & 1u))) {
      base += 1u; /* may carry into the exponent; 0x7c00 is +inf */
    }
    return (uint16_t)(sign | base);
  }
  /* subnormal half: k * 2^-24 with k = M * 2^(exponent + 1), M 24 bits */
  const int shift = -(exponent + 1);
  if (shift > 24) {
    return sign;
  }
  const uint32_t full = mantissa | 0x800000u;
  uint32_t k = full >> shift;
  const uint32_t rest = full & ((1u << shift) - 1u);
  const uint32_t half_point = 1u << (shift - 1);
  if (rest > half_point || (rest == half_point && (k & 1u))) {
    k += 1u;
  }
  return (uint16_t)(sign | k);
}

void orc_half_to_float_n(const uint16_t* in, float* out, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) {
    out[i] = orc_half_to_float(in[i]);
  }
}

/* ------------------------------------------------------------------------ */
/* Final RMSNorm: reference src/cpu/operators.cpp:523-535                    */
/*   sum_squares += value * value        (unfused, ascending columns)        */
/*   inverse = 1.0F / std::sqrt(sum_squares / float(hidden) + epsilon)       */
/*   output = input * inverse * weight   ((x * inv) * w)                     */
/* ------------------------------------------------------------------------ */

static float rms_inverse(const float* x, uint64_t hidden, float epsilon) {
  float sum_squares = 0.0f;
  for (uint64_t c = 0; c < hidden; ++c) {
    const float v = x[c];
    const float sq = v * v;
    sum_squares = sum_squares + sq;
  }
  const float mean = sum_squares / (float)hidden;
  return 1.0f / sqrtf(mean + epsilon);
}

void orc_rms_norm_f32(const float* input, const float* weight, float epsilon,
                      float* output, uint64_t rows, uint64_t hidden) {
  for (uint64_t r = 0; r < rows; ++r) {
    const float* x = input + r * hidden;
    float* y = output + r * hidden;
    const float inverse = rms_inverse(x, hidden, epsilon);
    for (uint64_t c = 0; c < hidden; ++c) {
      const float scaled = x[c] * inverse;
      y[c] = scaled * weight[c];
    }
  }
}

/* FP16 storage variant: the same FP32 arithmetic on decoded inputs, output
 * rounded to nearest-even half.  The reference GPU kernel
 * (src/cuda/rms_norm.cu:69-100) uses the same formula with an unspecified
 * rsqrtf; this build defines the FP16 op as the FP32 CPU order above. */
void orc_rms_norm_f16(const uint16_t* input, const uint16_t* weight,
                      float epsilon, uint16_t* output, uint64_t rows,
                      uint64_t hidden) {
  float* x = (float*)malloc(sizeof(float) * (hidden ? hidden : 1));
  for (uint64_t r = 0; r < rows; ++r) {
    for (uint64_t c = 0; c < hidden; ++c) {
      x[c] = orc_half_to_float(input[r * hidden + c]);
    }
    const float inverse = rms_inverse(x, hidden, epsilon);
    for (uint64_t c = 0; c < hidden; ++c) {
      const float scaled = x[c] * inverse;
      output[r * hidden + c] =
          orc_float_to_half(scaled * orc_half_to_float(weight[c]));
    }
  }
  free(x);
}

/* ------------------------------------------------------------------------ */
/* Dot products in the two reference orders                                  */
/* ------------------------------------------------------------------------ */

/* fmaf() is exactly rounded either way; the "fma" clone only replaces the
 * libm software routine by the hardware instruction where the host has it. */
#define ORC_FMA_CLONES __attribute__((target_clones("fma", "default")))

/* src/cuda/greedy.cu:171-176 and tests/cuda/cuda_tests.cu:739-744:
 *   score = fmaf(hidden[f], embedding[f], score), f ascending from 0. */
ORC_FMA_CLONES float orc_dot_fma(const float* hidden, const uint16_t* embedding_row,
                  uint64_t n) {
  float score = 0.0f;
  for (uint64_t f = 0; f < n; ++f) {
    score = fmaf(hidden[f], orc_half_to_float(embedding_row[f]), score);
  }
  return score;
}

/* src/cpu/operators.cpp:584-595 (linear_f32):
 *   sum += input[f] * weight[f]  (product rounded, then sum rounded). */
float orc_dot_mul_add(const float* hidden, const uint16_t* embedding_row,
                      uint64_t n) {
  float sum = 0.0f;
  for (uint64_t f = 0; f < n; ++f) {
    const float product = hidden[f] * orc_half_to_float(embedding_row[f]);
    sum = sum + product;
  }
  return sum;
}

static float dot_in_order(int order, const float* hidden,
                          const uint16_t* embedding_row, uint64_t n) {
  return order == ORC_ORDER_MUL_ADD_CHAIN
             ? orc_dot_mul_add(hidden, embedding_row, n)
             : orc_dot_fma(hidden, embedding_row, n);
}

/* The same two orders over an FP32 table (the FP32 CPU model,
 * src/cpu/smollm2.cpp:437-439, materializes FP32 weights). */
ORC_FMA_CLONES static float dot_in_order_f32(int order, const float* hidden,
                              const float* embedding_row, uint64_t n) {
  float s = 0.0f;
  if (order == ORC_ORDER_MUL_ADD_CHAIN) {
    for (uint64_t f = 0; f < n; ++f) {
      const float product = hidden[f] * embedding_row[f];
      s = s + product;
    }
  } else {
    for (uint64_t f = 0; f < n; ++f) {
      s = fmaf(hidden[f], embedding_row[f], s);
    }
  }
  return s;
}

typedef struct {
  const uint16_t* f16;
  const float* f32;
  uint64_t hidden;
  int order;
} orc_table;

static float table_dot(const orc_table* t, const float* y, uint64_t token) {
  if (t->f32) {
    return dot_in_order_f32(t->order, y, t->f32 + token * t->hidden, t->hidden);
  }
  return dot_in_order(t->order, y, t->f16 + token * t->hidden, t->hidden);
}

/* ------------------------------------------------------------------------ */
/* Selection rule: src/cuda/greedy.cu:84-100, 177-211                        */
/*   winner = lowest id among the maximal non-NaN scores (-0 == +0 ties);     */
/*   a set whose scores are all NaN falls back to its lowest id.             */
/* ------------------------------------------------------------------------ */

typedef struct {
  float best;
  uint32_t token;    /* ORC_INVALID_TOKEN until a non-NaN score is seen */
  uint32_t position; /* list position of token */
  uint32_t fallback; /* lowest id seen */
  uint32_t fallback_position;
} orc_selector;

static void selector_init(orc_selector* s) {
  s->best = -INFINITY;
  s->token = ORC_INVALID_TOKEN;
  s->position = 0;
  s->fallback = ORC_INVALID_TOKEN;
  s->fallback_position = 0;
}

static void selector_push(orc_selector* s, float score, uint32_t token,
                          uint32_t position) {
  if (token < s->fallback) {
    s->fallback = token;
    s->fallback_position = position;
  }
  if (score > s->best || (score == s->best && token < s->token)) {
    s->best = score;
    s->token = token;
    s->position = position;
  }
}

/* Returns the winner (fallback when every score was NaN) and its position. */
static uint32_t selector_result(const orc_selector* s, uint32_t* position,
                                int* all_nan) {
  if (s->token == ORC_INVALID_TOKEN) {
    *position = s->fallback_position;
    *all_nan = 1;
    return s->fallback;
  }
  *position = s->position;
  *all_nan = 0;
  return s->token;
}

/* ------------------------------------------------------------------------ */
/* Reference operators over FP16 tensors                                     */
/* ------------------------------------------------------------------------ */

/* greedy_kernel, src/cuda/greedy.cu:21-59: full-vocabulary argmax; a row with
 * no non-NaN value writes token 0 (greedy.cu:57). */
void orc_greedy_f16(const uint16_t* logits, uint64_t rows, uint64_t vocab,
                    uint32_t* token_ids) {
  for (uint64_t r = 0; r < rows; ++r) {
    float best = -INFINITY;
    uint32_t token = ORC_INVALID_TOKEN;
    for (uint64_t c = 0; c < vocab; ++c) {
      const float v = orc_half_to_float(logits[r * vocab + c]);
      if (v > best || (v == best && (uint32_t)c < token)) {
        best = v;
        token = (uint32_t)c;
      }
    }
    token_ids[r] = token == ORC_INVALID_TOKEN ? 0u : token;
  }
}

/* FP32-logit variants of the two selections above: identical rules applied to
 * binary32 values (the reference kernels read FP16 and widen to FP32 before
 * comparing, greedy.cu:32 and :95). */
void orc_greedy_f32(const float* logits, uint64_t rows, uint64_t vocab,
                    uint32_t* token_ids) {
  for (uint64_t r = 0; r < rows; ++r) {
    float best = -INFINITY;
    uint32_t token = ORC_INVALID_TOKEN;
    for (uint64_t c = 0; c < vocab; ++c) {
      const float v = logits[r * vocab + c];
      if (v > best || (v == best && (uint32_t)c < token)) {
        best = v;
        token = (uint32_t)c;
      }
    }
    token_ids[r] = token == ORC_INVALID_TOKEN ? 0u : token;
  }
}

void orc_restricted_greedy_f32(const float* logits, const uint32_t* allowed_ids,
                               const uint32_t* allowed_counts, uint64_t rows,
                               uint64_t vocab, uint64_t max_allowed,
                               uint32_t* token_ids) {
  for (uint64_t r = 0; r < rows; ++r) {
    const uint32_t count = allowed_counts[r];
    if (count == 0 || count > max_allowed) {
      token_ids[r] = ORC_INVALID_TOKEN;
      continue;
    }
    orc_selector s;
    selector_init(&s);
    int invalid = 0;
    for (uint32_t j = 0; j < count; ++j) {
      const uint32_t t = allowed_ids[r * max_allowed + j];
      if (t >= vocab) {
        invalid = 1;
        break;
      }
      selector_push(&s, logits[r * vocab + t], t, j);
    }
    uint32_t pos;
    int all_nan;
    token_ids[r] = invalid ? ORC_INVALID_TOKEN : selector_result(&s, &pos, &all_nan);
  }
}

/* restricted_greedy_kernel, src/cuda/greedy.cu:61-131. */
void orc_restricted_greedy_f16(const uint16_t* logits,
                               const uint32_t* allowed_ids,
                               const uint32_t* allowed_counts, uint64_t rows,
                               uint64_t vocab, uint64_t max_allowed,
                               uint32_t* token_ids) {
  for (uint64_t r = 0; r < rows; ++r) {
    const uint32_t count = allowed_counts[r];
    if (count == 0 || count > max_allowed) {
      token_ids[r] = ORC_INVALID_TOKEN;
      continue;
    }
    orc_selector s;
    selector_init(&s);
    int invalid = 0;
    for (uint32_t j = 0; j < count; ++j) {
      const uint32_t t = allowed_ids[r * max_allowed + j];
      if (t >= vocab) {
        invalid = 1;
        break;
      }
      selector_push(&s, orc_half_to_float(logits[r * vocab + t]), t, j);
    }
    uint32_t pos;
    int all_nan;
    token_ids[r] = invalid ? ORC_INVALID_TOKEN : selector_result(&s, &pos, &all_nan);
  }
}

/* restricted_output_head_kernel, src/cuda/greedy.cu:133-212: FP16 hidden and
 * embedding, sequential fmaf chain, same selection and sentinel rules. */
void orc_restricted_output_head_f16(const uint16_t* hidden,
                                    const uint16_t* embedding,
                                    const uint32_t* allowed_ids,
                                    const uint32_t* allowed_counts,
                                    uint64_t rows, uint64_t hidden_size,
                                    uint64_t vocab, uint64_t max_allowed,
                                    uint32_t* token_ids, float* scores) {
  float* h = (float*)malloc(sizeof(float) * (hidden_size ? hidden_size : 1));
  for (uint64_t r = 0; r < rows; ++r) {
    const uint32_t count = allowed_counts[r];
    if (scores) {
      scores[r] = NAN;
    }
    if (count == 0 || count > max_allowed) {
      token_ids[r] = ORC_INVALID_TOKEN;
      continue;
    }
    for (uint64_t f = 0; f < hidden_size; ++f) {
      h[f] = orc_half_to_float(hidden[r * hidden_size + f]);
    }
    orc_selector s;
    selector_init(&s);
    int invalid = 0;
    for (uint32_t j = 0; j < count; ++j) {
      const uint32_t t = allowed_ids[r * max_allowed + j];
      if (t >= vocab) {
        invalid = 1;
        break;
      }
      selector_push(&s, orc_dot_fma(h, embedding + (uint64_t)t * hidden_size,
                                    hidden_size),
                    t, j);
    }
    if (invalid) {
      token_ids[r] = ORC_INVALID_TOKEN;
      continue;
    }
    uint32_t pos;
    int all_nan;
    const uint32_t w = selector_result(&s, &pos, &all_nan);
    token_ids[r] = w;
    if (scores) {
      scores[r] = orc_dot_fma(h, embedding + (uint64_t)w * hidden_size,
                              hidden_size);
    }
  }
  free(h);
}

/* linear_f16 semantics (include/marketforge/cuda/linear.hpp:12-22): FP32
 * accumulation rounded to FP16.  The accumulation order follows the
 * reference test oracle, tests/cuda/cuda_tests.cu:170-181 (sequential fma). */
void orc_linear_f16(const uint16_t* input, const uint16_t* weight,
                    uint64_t rows, uint64_t in_features, uint64_t out_features,
                    uint16_t* output, float* output_f32) {
  float* x = (float*)malloc(sizeof(float) * (in_features ? in_features : 1));
  for (uint64_t r = 0; r < rows; ++r) {
    for (uint64_t f = 0; f < in_features; ++f) {
      x[f] = orc_half_to_float(input[r * in_features + f]);
    }
    for (uint64_t o = 0; o < out_features; ++o) {
      const float s = orc_dot_fma(x, weight + o * in_features, in_features);
      if (output) {
        output[r * out_features + o] = orc_float_to_half(s);
      }
      if (output_f32) {
        output_f32[r * out_features + o] = s;
      }
    }
  }
  free(x);
}

/* ------------------------------------------------------------------------ */
/* The north-star decode tail:                                               */
/*   RMSNorm (operators.cpp:523-535) -> scores of the state's allowed ids in */
/*   the chosen reference order -> greedy.cu selection -> DFA advance         */
/*   (token_dfa.cpp:111-128: the arc of the chosen token gives the next       */
/*   state; or a dense next table, -1 = disallowed).                          */
/* Row state conventions:                                                    */
/*   state < S                  restricted to the state's CSR list           */
/*   ORC_STATE_UNRESTRICTED     every token 0..V-1 (full-vocabulary row)      */
/*   anything else, an empty list or an out-of-vocabulary id -> token        */
/*   ORC_INVALID_TOKEN, next state ORC_INVALID_TOKEN, score NaN.              */
/* ------------------------------------------------------------------------ */

typedef struct {
  const float* x;
  const float* norm_weight; /* NULL: x is used as the normalized hidden */
  float epsilon;
  const uint16_t* embedding;
  const float* embedding_f32; /* FP32 table instead of FP16, or NULL */
  uint64_t vocab;
  uint64_t hidden;
  const uint32_t* row_state;
  uint64_t rows;
  const uint32_t* state_offsets;
  const uint32_t* state_tokens;
  uint64_t states;
  const uint32_t* state_next; /* parallel to state_tokens, or NULL */
  const int32_t* next_table;  /* [states, vocab], or NULL */
  int order;
  uint32_t* out_token;
  float* out_score;
  uint32_t* out_next;
  uint64_t row_begin;
  uint64_t row_end;
} orc_tail_job;

static void tail_rows(const orc_tail_job* job) {
  const uint64_t H = job->hidden;
  orc_table table;
  table.f16 = job->embedding;
  table.f32 = job->embedding_f32;
  table.hidden = H;
  table.order = job->order;
  float* y = (float*)malloc(sizeof(float) * (H ? H : 1));
  for (uint64_t r = job->row_begin; r < job->row_end; ++r) {
    const float* x = job->x + r * H;
    if (job->norm_weight) {
      const float inverse = rms_inverse(x, H, job->epsilon);
      for (uint64_t c = 0; c < H; ++c) {
        const float scaled = x[c] * inverse;
        y[c] = scaled * job->norm_weight[c];
      }
    } else {
      memcpy(y, x, sizeof(float) * H);
    }
    const uint32_t state = job->row_state[r];
    uint32_t token = ORC_INVALID_TOKEN;
    uint32_t next = ORC_INVALID_TOKEN;
    float score = NAN;
    if (state == ORC_STATE_UNRESTRICTED) {
      orc_selector s;
      selector_init(&s);
      for (uint64_t t = 0; t < job->vocab; ++t) {
        selector_push(&s, table_dot(&table, y, t), (uint32_t)t, (uint32_t)t);
      }
      uint32_t pos;
      int all_nan;
      token = selector_result(&s, &pos, &all_nan);
      score = all_nan ? NAN : s.best;
      next = ORC_STATE_UNRESTRICTED;
    } else if (state < job->states) {
      const uint32_t begin = job->state_offsets[state];
      const uint32_t end = job->state_offsets[state + 1];
      int invalid = end <= begin;
      orc_selector s;
      selector_init(&s);
      for (uint32_t j = begin; j < end && !invalid; ++j) {
        const uint32_t t = job->state_tokens[j];
        if (t >= job->vocab) {
          invalid = 1;
          break;
        }
        selector_push(&s, table_dot(&table, y, t), t, j - begin);
      }
      if (!invalid) {
        uint32_t pos;
        int all_nan;
        token = selector_result(&s, &pos, &all_nan);
        score = table_dot(&table, y, token);
        if (job->state_next) {
          next = job->state_next[begin + pos];
        } else if (job->next_table) {
          next = (uint32_t)job->next_table[(uint64_t)state * job->vocab + token];
        }
      }
    }
    job->out_token[r] = token;
    if (job->out_score) {
      job->out_score[r] = score;
    }
    if (job->out_next) {
      job->out_next[r] = next;
    }
  }
  free(y);
}

static void* tail_thread(void* arg) {
  tail_rows((const orc_tail_job*)arg);
  return NULL;
}

/* Multi-threaded over rows (threads <= 1 runs on the calling thread).  The
 * arithmetic per row is identical whatever the thread count. */
int orc_decode_tail(const float* x, const float* norm_weight, float epsilon,
                    const uint16_t* embedding, const float* embedding_f32,
                    uint64_t vocab, uint64_t hidden,
                    const uint32_t* row_state, uint64_t rows,
                    const uint32_t* state_offsets, const uint32_t* state_tokens,
                    uint64_t states, const uint32_t* state_next,
                    const int32_t* next_table, int order, uint32_t* out_token,
                    float* out_score, uint32_t* out_next, int threads) {
  orc_tail_job base;
  base.x = x;
  base.norm_weight = norm_weight;
  base.epsilon = epsilon;
  base.embedding = embedding;
  base.embedding_f32 = embedding_f32;
  base.vocab = vocab;
  base.hidden = hidden;
  base.row_state = row_state;
  base.rows = rows;
  base.state_offsets = state_offsets;
  base.state_tokens = state_tokens;
  base.states = states;
  base.state_next = state_next;
  base.next_table = next_table;
  base.order = order;
  base.out_token = out_token;
  base.out_score = out_score;
  base.out_next = out_next;
  if (threads <= 1 || rows < 2) {
    base.row_begin = 0;
    base.row_end = rows;
    tail_rows(&base);
    return 0;
  }
  if ((uint64_t)threads > rows) {
    threads = (int)rows;
  }
  pthread_t* ids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
  orc_tail_job* jobs = (orc_tail_job*)malloc(sizeof(orc_tail_job) * (size_t)threads);
  for (int i = 0; i < threads; ++i) {
    jobs[i] = base;
    jobs[i].row_begin = rows * (uint64_t)i / (uint64_t)threads;
    jobs[i].row_end = rows * (uint64_t)(i + 1) / (uint64_t)threads;
    if (pthread_create(&ids[i], NULL, tail_thread, &jobs[i]) != 0) {
      tail_rows(&jobs[i]);
      ids[i] = 0;
    }
  }
  for (int i = 0; i < threads; ++i) {
    if (ids[i]) {
      pthread_join(ids[i], NULL);
    }
  }
  free(ids);
  free(jobs);
  return 0;
}

/* Canonical scores of an explicit candidate list (used by tests to inspect
 * near-ties and by the brute-force cross-checks). */
void orc_scores(const float* hidden, const uint16_t* embedding,
                uint64_t hidden_size, const uint32_t* tokens, uint64_t n,
                int order, float* out) {
  for (uint64_t j = 0; j < n; ++j) {
    out[j] = dot_in_order(order, hidden,
                          embedding + (uint64_t)tokens[j] * hidden_size,
                          hidden_size);
  }
}
