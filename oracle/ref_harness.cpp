// TEST INFRASTRUCTURE ONLY: an extern "C" harness around the reference's own
// CPU sources, compiled in place from /root/reference by oracle/Makefile into
// oracle/_ref/libmfref.so.  It lets the tests check the oracle restatement
// (oracle/oracle.c) against the reference implementation, bit for bit.
//
// Wrapped reference entry points:
//   marketforge::rms_norm_f32   src/cpu/operators.cpp:489-537
//   marketforge::linear_f32     src/cpu/operators.cpp:539-597
//   marketforge::TokenDfa       src/grammar/token_dfa.cpp:23-148
//   SmolLm2MarketActionCatalog  src/grammar/smollm2_market_actions.cpp:42-73
#include <array>
#include <cstdint>
#include <span>
#include <vector>

#include "marketforge/core/shape.hpp"
#include "marketforge/core/tensor_view.hpp"
#include "marketforge/cpu/operators.hpp"
#include "marketforge/grammar/smollm2_market_actions.hpp"
#include "marketforge/grammar/token_dfa.hpp"

namespace {

marketforge::ConstTensorView const_view(const float* data,
                                        std::span<const std::uint64_t> dims) {
  return {data, marketforge::make_shape(dims).value(), marketforge::DType::f32,
          marketforge::MemoryKind::host};
}

marketforge::TensorView mut_view(float* data,
                                 std::span<const std::uint64_t> dims) {
  return {data, marketforge::make_shape(dims).value(), marketforge::DType::f32,
          marketforge::MemoryKind::host};
}

} // namespace

extern "C" {

int mfref_rms_norm_f32(const float* input, const float* weight, float epsilon,
                       float* output, std::uint64_t rows,
                       std::uint64_t hidden) {
  const std::array<std::uint64_t, 2> dims{rows, hidden};
  const std::array<std::uint64_t, 1> wdims{hidden};
  return static_cast<int>(marketforge::rms_norm_f32(const_view(input, dims),
                                                    const_view(weight, wdims),
                                                    epsilon,
                                                    mut_view(output, dims))
                              .code);
}

int mfref_linear_f32(const float* input, const float* weight, float* output,
                     std::uint64_t rows, std::uint64_t in_features,
                     std::uint64_t out_features) {
  const std::array<std::uint64_t, 2> idims{rows, in_features};
  const std::array<std::uint64_t, 2> wdims{out_features, in_features};
  const std::array<std::uint64_t, 2> odims{rows, out_features};
  return static_cast<int>(marketforge::linear_f32(const_view(input, idims),
                                                  const_view(weight, wdims),
                                                  mut_view(output, odims))
                              .code);
}

// Builds a TokenDfa from flattened choices and exports its states as CSR:
// offsets[states + 1], arc tokens / next states [arcs], terminal choice id per
// state (UINT32_MAX when not terminal).  Returns the build's error code, or 0
// and writes counts.  Capacity arguments bound every output array.
int mfref_token_dfa_export(const std::uint32_t* choice_ids,
                           const std::uint32_t* token_offsets,
                           const std::uint32_t* tokens,
                           std::uint32_t choice_count,
                           std::uint32_t vocabulary_size,
                           std::uint32_t maximum_sequence_tokens,
                           std::uint32_t maximum_choices,
                           std::uint32_t maximum_states,
                           std::uint32_t maximum_arcs,
                           std::uint32_t* out_offsets,
                           std::uint32_t* out_tokens, std::uint32_t* out_next,
                           std::uint32_t* out_terminal,
                           std::uint32_t state_capacity,
                           std::uint32_t arc_capacity,
                           std::uint32_t* out_states,
                           std::uint32_t* out_arcs) {
  std::vector<marketforge::EncodedChoice> language;
  for (std::uint32_t c = 0; c < choice_count; ++c) {
    marketforge::EncodedChoice choice;
    choice.id = choice_ids[c];
    for (std::uint32_t i = token_offsets[c]; i < token_offsets[c + 1]; ++i) {
      choice.tokens.push_back(tokens[i]);
    }
    language.push_back(std::move(choice));
  }
  const marketforge::TokenDfaConfig config{vocabulary_size,
                                           maximum_sequence_tokens,
                                           maximum_choices, maximum_states,
                                           maximum_arcs};
  auto built = marketforge::TokenDfa::build(language, config);
  if (!built) {
    return static_cast<int>(built.status().code);
  }
  const auto& dfa = built.value();
  const auto states = static_cast<std::uint32_t>(dfa.state_count());
  const auto arcs = static_cast<std::uint32_t>(dfa.arc_count());
  *out_states = states;
  *out_arcs = arcs;
  if (states + 1 > state_capacity || arcs > arc_capacity) {
    return -1;
  }
  std::uint32_t cursor = 0;
  for (std::uint32_t s = 0; s < states; ++s) {
    out_offsets[s] = cursor;
    const auto allowed = dfa.allowed(marketforge::GrammarState{s}).value();
    for (const auto& arc : allowed) {
      out_tokens[cursor] = arc.token;
      out_next[cursor] = arc.next.value;
      ++cursor;
    }
    const auto decoded = dfa.decode_terminal(marketforge::GrammarState{s});
    out_terminal[s] = decoded ? decoded.value() : UINT32_MAX;
  }
  out_offsets[states] = cursor;
  return 0;
}

// Reference TokenDfa::advance on a freshly built DFA (same inputs as above):
// returns the error code, writes the next state.
int mfref_token_dfa_advance(const std::uint32_t* choice_ids,
                            const std::uint32_t* token_offsets,
                            const std::uint32_t* tokens,
                            std::uint32_t choice_count,
                            std::uint32_t vocabulary_size,
                            std::uint32_t state, std::uint32_t token,
                            std::uint32_t* next) {
  std::vector<marketforge::EncodedChoice> language;
  for (std::uint32_t c = 0; c < choice_count; ++c) {
    marketforge::EncodedChoice choice;
    choice.id = choice_ids[c];
    for (std::uint32_t i = token_offsets[c]; i < token_offsets[c + 1]; ++i) {
      choice.tokens.push_back(tokens[i]);
    }
    language.push_back(std::move(choice));
  }
  marketforge::TokenDfaConfig config{};
  config.vocabulary_size = vocabulary_size;
  auto built = marketforge::TokenDfa::build(language, config);
  if (!built) {
    return static_cast<int>(built.status().code);
  }
  const auto advanced =
      built.value().advance(marketforge::GrammarState{state}, token);
  if (!advanced) {
    return static_cast<int>(advanced.status().code);
  }
  *next = advanced.value().value;
  return 0;
}

// Exports the SmolLM2 market-action DFA (src/grammar/generated data) as CSR,
// plus per state the index of its terminal action in catalog.entries()
// (UINT32_MAX when not terminal; out_terminal may be null).
int mfref_market_dfa_export(std::uint32_t* out_offsets,
                            std::uint32_t* out_tokens, std::uint32_t* out_next,
                            std::uint32_t* out_terminal,
                            std::uint32_t state_capacity,
                            std::uint32_t arc_capacity,
                            std::uint32_t* out_states,
                            std::uint32_t* out_arcs) {
  auto catalog = marketforge::SmolLm2MarketActionCatalog::create();
  if (!catalog) {
    return static_cast<int>(catalog.status().code);
  }
  const auto& dfa = catalog.value().dfa();
  const auto states = static_cast<std::uint32_t>(dfa.state_count());
  const auto arcs = static_cast<std::uint32_t>(dfa.arc_count());
  *out_states = states;
  *out_arcs = arcs;
  if (states + 1 > state_capacity || arcs > arc_capacity) {
    return -1;
  }
  std::uint32_t cursor = 0;
  for (std::uint32_t s = 0; s < states; ++s) {
    out_offsets[s] = cursor;
    const auto allowed = dfa.allowed(marketforge::GrammarState{s}).value();
    for (const auto& arc : allowed) {
      out_tokens[cursor] = arc.token;
      out_next[cursor] = arc.next.value;
      ++cursor;
    }
    if (out_terminal != nullptr) {
      out_terminal[s] = UINT32_MAX;
      const auto decoded = dfa.decode_terminal(marketforge::GrammarState{s});
      if (decoded) {
        const auto entries = catalog.value().entries();
        for (std::uint32_t i = 0; i < entries.size(); ++i) {
          if (entries[i].action == decoded.value()) {
            out_terminal[s] = i;
            break;
          }
        }
      }
    }
  }
  out_offsets[states] = cursor;
  return 0;
}

// The market-action language: token sequence of every catalog entry, as
// offsets[entries + 1] into tokens.
int mfref_market_language(std::uint32_t* out_offsets, std::uint32_t* out_tokens,
                          std::uint32_t entry_capacity, std::uint32_t token_capacity,
                          std::uint32_t* out_entries, std::uint32_t* out_token_count) {
  auto catalog = marketforge::SmolLm2MarketActionCatalog::create();
  if (!catalog) {
    return static_cast<int>(catalog.status().code);
  }
  const auto entries = catalog.value().entries();
  std::uint32_t n = 0;
  for (const auto& e : entries) n += static_cast<std::uint32_t>(e.tokens.size());
  *out_entries = static_cast<std::uint32_t>(entries.size());
  *out_token_count = n;
  if (entries.size() + 1 > entry_capacity || n > token_capacity) {
    return -1;
  }
  std::uint32_t cursor = 0;
  for (std::uint32_t i = 0; i < entries.size(); ++i) {
    out_offsets[i] = cursor;
    for (const auto t : entries[i].tokens) out_tokens[cursor++] = t;
  }
  out_offsets[entries.size()] = cursor;
  return 0;
}

} // extern "C"
