/*
 * Host sanitizer run of the CPU oracle (oracle/oracle.c), test
 * infrastructure: built with -fsanitize=address,undefined and
 * -fno-sanitize-recover=all by tests/cpp/Makefile (target `sanitize`), so an
 * out-of-bounds access, a use after free, a signed overflow or a bad shift
 * in the oracle ends the run with a report.
 *
 * Every exported function is called on small seeded inputs, with the edge
 * cases the decode tail has (unrestricted rows, invalid states, empty
 * lists, ids past the vocabulary, NaN hidden rows, a next table and an arc
 * table, both orders, the FP16 and the FP32 table, 1 and 4 threads), and
 * the runs that must agree are compared, so the driver also fails on a
 * result that depends on the thread count or the table's storage.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

float orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float f);
void orc_half_to_float_n(const uint16_t* in, float* out, uint64_t n);
void orc_rms_norm_f32(const float* input, const float* weight, float epsilon, float* output,
                      uint64_t rows, uint64_t hidden);
void orc_rms_norm_f16(const uint16_t* input, const uint16_t* weight, float epsilon,
                      uint16_t* output, uint64_t rows, uint64_t hidden);
float orc_dot_fma(const float* hidden, const uint16_t* embedding_row, uint64_t n);
float orc_dot_mul_add(const float* hidden, const uint16_t* embedding_row, uint64_t n);
void orc_greedy_f16(const uint16_t* logits, uint64_t rows, uint64_t vocab, uint32_t* token_ids);
void orc_greedy_f32(const float* logits, uint64_t rows, uint64_t vocab, uint32_t* token_ids);
void orc_restricted_greedy_f32(const float* logits, const uint32_t* allowed_ids,
                               const uint32_t* allowed_counts, uint64_t rows, uint64_t vocab,
                               uint64_t max_allowed, uint32_t* token_ids);
void orc_restricted_greedy_f16(const uint16_t* logits, const uint32_t* allowed_ids,
                               const uint32_t* allowed_counts, uint64_t rows, uint64_t vocab,
                               uint64_t max_allowed, uint32_t* token_ids);
void orc_restricted_output_head_f16(const uint16_t* hidden, const uint16_t* embedding,
                                    const uint32_t* allowed_ids, const uint32_t* allowed_counts,
                                    uint64_t rows, uint64_t hidden_size, uint64_t vocab,
                                    uint64_t max_allowed, uint32_t* token_ids, float* scores);
void orc_linear_f16(const uint16_t* input, const uint16_t* weight, uint64_t rows,
                    uint64_t in_features, uint64_t out_features, uint16_t* output,
                    float* output_f32);
int orc_decode_tail(const float* x, const float* norm_weight, float epsilon,
                    const uint16_t* embedding, const float* embedding_f32, uint64_t vocab,
                    uint64_t hidden, const uint32_t* row_state, uint64_t rows,
                    const uint32_t* state_offsets, const uint32_t* state_tokens,
                    uint64_t states, const uint32_t* state_next, const int32_t* next_table,
                    int order, uint32_t* out_token, float* out_score, uint32_t* out_next,
                    int threads);
void orc_scores(const float* hidden, const uint16_t* embedding, uint64_t hidden_size,
                const uint32_t* tokens, uint64_t n, int order, float* out);

static int failures = 0;
static int checks = 0;

static void check(int ok, const char* what) {
  ++checks;
  if (!ok) {
    ++failures;
    printf("FAIL: %s\n", what);
  }
}

/* splitmix64: a seeded stream for the inputs */
static uint64_t g_state = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64(void) {
  uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
static float uniform_pm1(void) { return (float)((double)(next_u64() >> 11) * 0x1p-53 * 2.0 - 1.0); }
static uint32_t below(uint32_t n) { return (uint32_t)(next_u64() % n); }

static void* xmalloc(size_t n) {
  void* p = malloc(n ? n : 1);
  if (!p) {
    printf("out of memory\n");
    exit(2);
  }
  return p;
}

static int same_bits_f32(const float* a, const float* b, uint64_t n) {
  return memcmp(a, b, n * sizeof(float)) == 0;
}

static void halves_and_norms(void) {
  for (uint32_t h = 0; h < 65536u; ++h) {
    const float f = orc_half_to_float((uint16_t)h);
    if (f == f) check(orc_float_to_half(f) == (uint16_t)h, "half round trip");
  }
  const uint64_t rows = 5, H = 33;
  float* x = xmalloc(rows * H * sizeof(float));
  float* w = xmalloc(H * sizeof(float));
  float* y = xmalloc(rows * H * sizeof(float));
  uint16_t* x16 = xmalloc(rows * H * 2);
  uint16_t* w16 = xmalloc(H * 2);
  uint16_t* y16 = xmalloc(rows * H * 2);
  for (uint64_t i = 0; i < rows * H; ++i) x[i] = uniform_pm1() * 3.0f;
  for (uint64_t i = 0; i < H; ++i) w[i] = 1.0f + 0.02f * uniform_pm1();
  x[2 * H + 4] = NAN;
  for (uint64_t i = 0; i < rows * H; ++i) x16[i] = orc_float_to_half(x[i]);
  for (uint64_t i = 0; i < H; ++i) w16[i] = orc_float_to_half(w[i]);
  orc_rms_norm_f32(x, w, 1e-5f, y, rows, H);
  orc_rms_norm_f16(x16, w16, 1e-5f, y16, rows, H);
  check(isnan(y[2 * H]), "a NaN input makes its row NaN");
  check(isfinite(y[0]) && isfinite(orc_half_to_float(y16[0])), "finite rows stay finite");
  float* dec = xmalloc(H * sizeof(float));
  orc_half_to_float_n(x16, dec, H);
  check(dec[0] == orc_half_to_float(x16[0]) && dec[H - 1] == orc_half_to_float(x16[H - 1]),
        "bulk decode equals scalar decode");
  free(x);
  free(w);
  free(y);
  free(x16);
  free(w16);
  free(y16);
  free(dec);
}

static void selections_and_linear(void) {
  const uint64_t rows = 6, V = 41, maxa = 7, H = 24;
  float* lg = xmalloc(rows * V * sizeof(float));
  uint16_t* lg16 = xmalloc(rows * V * 2);
  for (uint64_t i = 0; i < rows * V; ++i) {
    lg[i] = uniform_pm1();
    lg16[i] = orc_float_to_half(lg[i]);
  }
  for (uint64_t c = 0; c < V; ++c) lg[3 * V + c] = NAN; /* an all-NaN row */
  lg[1 * V + 9] = lg[1 * V + 10] = 5.0f;                 /* a tie */
  uint32_t ids[6 * 7];
  uint32_t counts[6] = {3, 0, 7, 8, 1, 7};               /* 0 and > max: invalid */
  for (uint64_t i = 0; i < rows * maxa; ++i) ids[i] = below((uint32_t)V);
  ids[5 * maxa + 2] = (uint32_t)V + 3;                  /* an id past the vocabulary */
  uint32_t t1[6], t2[6], t3[6], t4[6];
  orc_greedy_f32(lg, rows, V, t1);
  orc_greedy_f16(lg16, rows, V, t2);
  orc_restricted_greedy_f32(lg, ids, counts, rows, V, maxa, t3);
  orc_restricted_greedy_f16(lg16, ids, counts, rows, V, maxa, t4);
  check(t1[1] == 9, "greedy tie -> lower id");
  check(t3[1] == 0xFFFFFFFFu && t3[3] == 0xFFFFFFFFu, "count 0 and count > max -> sentinel");
  check(t4[1] == 0xFFFFFFFFu && t4[3] == 0xFFFFFFFFu, "f16 sentinel rows");

  uint16_t* hid = xmalloc(rows * H * 2);
  uint16_t* emb = xmalloc(V * H * 2);
  for (uint64_t i = 0; i < rows * H; ++i) hid[i] = orc_float_to_half(uniform_pm1());
  for (uint64_t i = 0; i < V * H; ++i) emb[i] = orc_float_to_half(0.1f * uniform_pm1());
  uint32_t ht[6];
  float hs[6];
  orc_restricted_output_head_f16(hid, emb, ids, counts, rows, H, V, maxa, ht, hs);
  check(ht[1] == 0xFFFFFFFFu, "head: count 0 -> sentinel");
  check(ht[5] == 0xFFFFFFFFu, "head: id past the vocabulary -> sentinel");
  uint16_t* out = xmalloc(rows * V * 2);
  float* out32 = xmalloc(rows * V * sizeof(float));
  orc_linear_f16(hid, emb, rows, H, V, out, out32);
  float hf[24];
  for (uint64_t f = 0; f < H; ++f) hf[f] = orc_half_to_float(hid[2 * H + f]);
  check(out32[2 * V + 11] == orc_dot_mul_add(hf, emb + 11 * H, H), "linear = mul-add dot");
  float sc[2];
  uint32_t tk[2] = {3, 40};
  orc_scores(hf, emb, H, tk, 2, 0, sc);
  check(sc[0] == orc_dot_fma(hf, emb + 3 * H, H) && sc[1] == orc_dot_fma(hf, emb + 40 * H, H),
        "orc_scores = fma dot");
  free(lg);
  free(lg16);
  free(hid);
  free(emb);
  free(out);
  free(out32);
}

static void decode_tail(void) {
  const uint64_t V = 700, H = 48, rows = 37, S = 9;
  uint16_t* emb = xmalloc(V * H * 2);
  float* emb32 = xmalloc(V * H * sizeof(float));
  for (uint64_t i = 0; i < V * H; ++i) {
    emb[i] = orc_float_to_half(0.02f * uniform_pm1());
    emb32[i] = orc_half_to_float(emb[i]);
  }
  float* x = xmalloc(rows * H * sizeof(float));
  float* w = xmalloc(H * sizeof(float));
  for (uint64_t i = 0; i < rows * H; ++i) x[i] = uniform_pm1();
  for (uint64_t i = 0; i < H; ++i) w[i] = 1.0f + 0.02f * uniform_pm1();
  for (uint64_t f = 0; f < H; ++f) x[7 * H + f] = NAN;
  uint32_t offsets[10];
  uint32_t* tokens = xmalloc(S * 300 * sizeof(uint32_t));
  uint32_t* nexts = xmalloc(S * 300 * sizeof(uint32_t));
  int32_t* table = xmalloc(S * V * sizeof(int32_t));
  for (uint64_t i = 0; i < S * V; ++i) table[i] = -1;
  offsets[0] = 0;
  for (uint32_t s = 0; s < S; ++s) {
    const uint32_t n = s == 4 ? 0u : 1u + below(250); /* state 4: an empty list */
    uint32_t at = offsets[s];
    for (uint32_t j = 0; j < n; ++j) {
      uint32_t t = below((uint32_t)V);
      int dup = 0;
      for (uint32_t k = offsets[s]; k < at; ++k) dup |= tokens[k] == t;
      if (dup) continue;
      tokens[at] = t;
      nexts[at] = below((uint32_t)S);
      table[(uint64_t)s * V + t] = (int32_t)nexts[at];
      ++at;
    }
    offsets[s + 1] = at;
  }
  tokens[offsets[6]] = (uint32_t)V + 1; /* state 6 holds an id past the vocabulary */
  uint32_t state[37];
  for (uint64_t r = 0; r < rows; ++r) state[r] = below((uint32_t)S);
  state[3] = 0xFFFFFFFEu; /* unrestricted */
  state[5] = 0xFFFFFFFEu;
  state[9] = (uint32_t)S + 2; /* invalid state */
  state[11] = 4;
  state[13] = 6;
  uint32_t tok[4][37], nx[4][37];
  float sc[4][37];
  for (int order = 0; order < 2; ++order) {
    orc_decode_tail(x, w, 1e-5f, emb, NULL, V, H, state, rows, offsets, tokens, S, nexts, NULL,
                    order, tok[0], sc[0], nx[0], 1);
    orc_decode_tail(x, w, 1e-5f, emb, NULL, V, H, state, rows, offsets, tokens, S, nexts, NULL,
                    order, tok[1], sc[1], nx[1], 4);
    orc_decode_tail(x, w, 1e-5f, NULL, emb32, V, H, state, rows, offsets, tokens, S, nexts, NULL,
                    order, tok[2], sc[2], nx[2], 3);
    orc_decode_tail(x, w, 1e-5f, emb, NULL, V, H, state, rows, offsets, tokens, S, NULL, table,
                    order, tok[3], sc[3], nx[3], 4);
    for (int k = 1; k < 4; ++k) {
      check(memcmp(tok[0], tok[k], sizeof(tok[0])) == 0, "tokens independent of threads/table");
      check(same_bits_f32(sc[0], sc[k], rows), "scores independent of threads/table");
    }
    check(memcmp(nx[0], nx[1], sizeof(nx[0])) == 0 && memcmp(nx[0], nx[2], sizeof(nx[0])) == 0,
          "next states independent of threads/table");
    for (uint64_t r = 0; r < rows; ++r) {
      if (tok[0][r] != 0xFFFFFFFFu && state[r] < S) {
        check(nx[0][r] == nx[3][r], "arc advance = next table advance");
      }
    }
    check(tok[0][9] == 0xFFFFFFFFu && nx[0][9] == 0xFFFFFFFFu, "invalid state");
    check(tok[0][11] == 0xFFFFFFFFu, "empty list -> invalid");
    check(tok[0][13] == 0xFFFFFFFFu, "id past the vocabulary -> invalid");
    check(nx[0][3] == 0xFFFFFFFEu && tok[0][3] < V, "unrestricted row");
  }
  /* no norm weight, no score or next-state outputs */
  orc_decode_tail(x, NULL, 1e-5f, emb, NULL, V, H, state, rows, offsets, tokens, S, NULL, NULL, 0,
                  tok[0], NULL, NULL, 2);
  check(tok[0][9] == 0xFFFFFFFFu, "optional outputs absent");
  free(emb);
  free(emb32);
  free(x);
  free(w);
  free(tokens);
  free(nexts);
  free(table);
}

int main(void) {
  halves_and_norms();
  selections_and_linear();
  decode_tail();
  printf("oracle_sanitize: %d checks, %d failures\n", checks, failures);
  return failures == 0 ? 0 : 1;
}
