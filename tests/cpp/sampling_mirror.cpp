// Drives justfit::hip::Sampling (the C++ mirror of the reference's
// ops::Sampling) the way the engine does, and prints its results as JSON.
//   sampling_mirror cpu   argument checks and host helpers (no GPU)
//   sampling_mirror gpu   addInitial, addVerify and addAcceptance on
//                         deterministic inputs (tests/test_cpp_mirror.py
//                         rebuilds the same inputs and checks the results
//                         against the CPU oracle)
//   sampling_mirror verify16  the widest verify step: 4 lanes x 16 rows at
//                         V = 248,320 (one selection call), then acceptance
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "sampling.hpp"

using namespace justfit::hip;

namespace {

int failures = 0;

#define EXPECT(cond)                                                  \
  do {                                                                \
    if (!(cond)) {                                                    \
      std::fprintf(stderr, "FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond); \
      ++failures;                                                     \
    }                                                                 \
  } while (0)

template <class E, class F>
bool throws(F f) {
  try {
    f();
  } catch (const E &) {
    return true;
  } catch (...) {
    return false;
  }
  return false;
}

void hip(hipError_t e) {
  if (e != hipSuccess) throw std::runtime_error(hipGetErrorString(e));
}

// The deterministic inputs, restated in tests/test_cpp_mirror.py.
constexpr uint32_t V = 1000;
float logit(uint32_t row, uint32_t t) {
  return (float)(((t * 7919ull + row * 104729ull) % 2003ull) / 200.0 - 5.0);
}
float uniform(uint32_t lane, uint32_t slot) {
  return (float)(((lane * 40ull + slot) * 37ull % 101ull) / 101.0);
}

int cpu_checks() {
  EXPECT(throws<std::invalid_argument>([] { Sampling s(0); }));
  EXPECT(activeVerifyRows() == 8);
  {
    VerifyShapeScope scope(16);
    EXPECT(activeVerifyRows() == 16);
    EXPECT(throws<std::invalid_argument>([] { VerifyShapeScope bad(9); }));
  }
  EXPECT(activeVerifyRows() == 8);
  // rebuildPenaltyWords: prompt ids 3, 3, 7 then generated 7, 9 and a
  // pending 9 (Sampling.cpp:50-71): prompt bits on 3 and 7, counts 7:1, 9:2.
  std::vector<uint32_t> words(16, 123u);
  const std::vector<uint32_t> history{3, 3, 7, 7, 9};
  Sampling::rebuildPenaltyWords(words, history, 2, 9u, true);
  EXPECT(words[3] == JF_PENALTY_PROMPT_BIT);
  EXPECT(words[7] == (JF_PENALTY_PROMPT_BIT | 1u));
  EXPECT(words[9] == 2u);
  EXPECT(words[0] == 0u && words[15] == 0u);
  Sampling::countPenaltyTokens(words, std::vector<uint32_t>{9, 3});
  EXPECT(words[9] == 3u);
  EXPECT(words[3] == (JF_PENALTY_PROMPT_BIT | 1u));
  // The reference checks for a prompt first (logic_error), then the ids.
  EXPECT(throws<std::logic_error>([&] {
    Sampling::rebuildPenaltyWords(words, std::vector<uint32_t>{16}, 1, std::nullopt, false);
  }));
  EXPECT(!throws<std::invalid_argument>([&] {
    Sampling::rebuildPenaltyWords(words, std::vector<uint32_t>{16}, 1, std::nullopt, false);
  }));
  EXPECT(throws<std::invalid_argument>([&] {
    Sampling::rebuildPenaltyWords(words, std::vector<uint32_t>{2, 16}, 1, std::nullopt, false);
  }));
  EXPECT(throws<std::invalid_argument>([&] {
    Sampling::rebuildPenaltyWords(words, std::vector<uint32_t>{2, 3}, 1, 16u, false);
  }));
  EXPECT(throws<std::invalid_argument>([&] {
    Sampling::countPenaltyTokens(words, std::vector<uint32_t>{99});
  }));
  std::printf("{\"cpu_failures\": %d}\n", failures);
  return failures ? 1 : 0;
}

template <class T>
DeviceBuffer upload(const std::vector<T> &host) {
  DeviceBuffer b;
  b.sizeBytes = host.size() * sizeof(T);
  hip(hipMalloc(&b.data, b.sizeBytes));
  hip(hipMemcpy(b.data, host.data(), b.sizeBytes, hipMemcpyHostToDevice));
  return b;
}
template <class T>
std::vector<T> download(const DeviceBuffer &b) {
  std::vector<T> host(b.sizeBytes / sizeof(T));
  hip(hipMemcpy(host.data(), b.data, b.sizeBytes, hipMemcpyDeviceToHost));
  return host;
}

void print_u32(const char *name, const std::vector<uint32_t> &v, bool comma = true) {
  std::printf("\"%s\": [", name);
  for (size_t i = 0; i < v.size(); ++i) std::printf("%s%u", i ? ", " : "", v[i]);
  std::printf("]%s\n", comma ? "," : "");
}
void print_f32(const char *name, const std::vector<float> &v, bool comma = true) {
  std::printf("\"%s\": [", name);
  for (size_t i = 0; i < v.size(); ++i) {
    uint32_t bits;
    std::memcpy(&bits, &v[i], 4);
    std::printf("%s%u", i ? ", " : "", bits);
  }
  std::printf("]%s\n", comma ? "," : "");
}

int gpu_checks() {
  const uint32_t rows = activeVerifyRows();  // 8
  const uint32_t lanes = 2;
  Sampling sampling(V, lanes);
  hipStream_t stream;
  hip(hipStreamCreate(&stream));

  std::vector<float> logits((size_t)lanes * rows * V);
  for (uint32_t r = 0; r < lanes * rows; ++r)
    for (uint32_t t = 0; t < V; ++t) logits[(size_t)r * V + t] = logit(r, t);
  std::vector<float> uniforms(lanes * JF_SAMPLING_UNIFORMS);
  for (uint32_t l = 0; l < lanes; ++l)
    for (uint32_t s = 0; s < JF_SAMPLING_UNIFORMS; ++s)
      uniforms[l * JF_SAMPLING_UNIFORMS + s] = uniform(l, s);
  // Lane 1's inputs: the anchor then seven draft tokens; candidate 0 of
  // each drafted row is its draft token.
  std::vector<uint32_t> inputs((size_t)lanes * rows);
  for (uint32_t i = 0; i < lanes * rows; ++i) inputs[i] = (i * 131u + 17u) % V;
  std::vector<uint32_t> cands((size_t)lanes * (rows - 1) * 16);
  std::vector<float> cprobs(cands.size());
  for (uint32_t l = 0; l < lanes; ++l)
    for (uint32_t r = 0; r + 1 < rows; ++r)
      for (uint32_t j = 0; j < 16; ++j) {
        const size_t k = ((size_t)l * (rows - 1) + r) * 16 + j;
        cands[k] = j ? (r * 53u + j * 97u) % V : inputs[l * rows + r + 1];
        cprobs[k] = j ? 0.02f : 0.7f;
      }

  jf_penalty_table *table = nullptr;
  if (jf_penalty_table_create(V, lanes, 64, &table) != JF_OK)
    throw std::runtime_error(jf_last_error());
  const std::vector<uint32_t> history{5, 17, 17, 999};
  if (jf_penalty_table_rebuild(table, 0, history.data(), history.size(), 2, 0, 0, 1,
                               stream) != JF_OK)
    throw std::runtime_error(jf_last_error());
  const std::vector<uint32_t> stateLanes{0, 1};

  SamplingBuffers b;
  b.logits = upload(logits);
  b.uniforms = upload(uniforms);
  b.inputTokens = upload(inputs);
  b.draftCandidates = upload(cands);
  b.draftProbabilities = upload(cprobs);
  b.outputTokens = upload(std::vector<uint32_t>((size_t)lanes * rows, 0));
  b.targetProbabilities = upload(std::vector<float>((size_t)lanes * rows, 0.0f));

  SamplingPolicy greedy;
  greedy.penalties.repetition = 1.2f;
  SamplingPolicy sampled;
  sampled.temperature = 0.8f;
  sampled.topK = 30;
  sampled.topP = 0.9f;
  const std::vector<SamplingPolicy> initial{greedy, sampled};
  // Lane 0 reads table row 0; lane 1's policy has no penalties.
  sampling.addInitial(stream, initial, b, 0, JF_NO_TOKEN, JF_NO_TOKEN,
                      PenaltyTable{table, stateLanes});
  hip(hipStreamSynchronize(stream));
  const std::vector<uint32_t> initialTokens = download<uint32_t>(b.outputTokens);

  // A too-small logits buffer is rejected before anything is enqueued.
  SamplingBuffers small = b;
  small.logits.sizeBytes = 16;
  EXPECT(throws<std::invalid_argument>([&] {
    sampling.addInitial(stream, initial, small, 0, JF_NO_TOKEN, JF_NO_TOKEN,
                        PenaltyTable{table, stateLanes});
  }));

  SamplingPolicy verify;
  verify.temperature = 1.0f;
  verify.topK = 50;
  verify.penalties.presence = 0.3f;
  const std::vector<SamplingPolicy> verifyPolicies{verify, verify};
  sampling.addVerify(stream, verifyPolicies, b, JF_NO_TOKEN, JF_NO_TOKEN,
                     PenaltyTable{table, stateLanes});
  hip(hipStreamSynchronize(stream));
  const std::vector<uint32_t> verifyTokens = download<uint32_t>(b.outputTokens);
  const std::vector<float> verifyProbs = download<float>(b.targetProbabilities);

  // Acceptance of both lanes' chains (proposals = inputs rows 1..7).
  std::vector<uint32_t> proposed((size_t)lanes * (rows - 1));
  for (uint32_t l = 0; l < lanes; ++l)
    for (uint32_t r = 0; r + 1 < rows; ++r)
      proposed[l * (rows - 1) + r] = inputs[l * rows + r + 1];
  AcceptanceBuffers ab;
  ab.proposedTokens = upload(proposed);
  ab.candidates = b.draftCandidates;
  ab.proposalProbabilities = b.draftProbabilities;
  ab.targetProbabilities = b.targetProbabilities;
  ab.uniforms = b.uniforms;
  ab.outputTokens = b.outputTokens;
  ab.retainedCounts = upload(std::vector<uint32_t>(lanes, 0));
  ab.acceptedCounts = upload(std::vector<uint32_t>(lanes, 0));
  const std::vector<uint32_t> maximumRetained{8, 5};
  sampling.addAcceptance(stream, ab, maximumRetained, verifyPolicies, JF_NO_TOKEN,
                         JF_NO_TOKEN);
  hip(hipStreamSynchronize(stream));
  const std::vector<uint32_t> accepted = download<uint32_t>(ab.outputTokens);
  const std::vector<uint32_t> retained = download<uint32_t>(ab.retainedCounts);
  const std::vector<uint32_t> acceptedCounts = download<uint32_t>(ab.acceptedCounts);

  std::printf("{\n");
  print_u32("initial_tokens", initialTokens);
  print_u32("verify_tokens", verifyTokens);
  print_f32("verify_probs_bits", verifyProbs);
  print_u32("accepted_tokens", accepted);
  print_u32("retained", retained);
  print_u32("accepted", acceptedCounts);
  std::printf("\"gpu_failures\": %d\n}\n", failures);
  jf_penalty_table_destroy(table);
  for (DeviceBuffer *d : {&b.logits, &b.uniforms, &b.inputTokens, &b.draftCandidates,
                          &b.draftProbabilities, &b.outputTokens, &b.targetProbabilities,
                          &ab.proposedTokens, &ab.retainedCounts, &ab.acceptedCounts})
    hip(hipFree(d->data));
  hip(hipStreamDestroy(stream));
  return failures ? 1 : 0;
}

// The engine's widest verify step: 4 lanes x 16 rows at V = 248,320, two
// lanes penalized (their verify rows count input rows 1..r on top of the
// table), sparse drafts; addVerify (correction uniform) and addVerify with
// tree draws (uniform 24 + r), then addAcceptance of the first. Inputs are
// restated in tests/test_cpp_mirror.py.
constexpr uint32_t V16 = 248320;
float logit16(uint32_t row, uint32_t t) {
  return (float)(((t * 48271ull + row * 16807ull) % 10007ull) / 1000.0 - 5.0);
}

int gpu_verify16() {
  VerifyShapeScope shape(16);
  const uint32_t rows = activeVerifyRows();
  const uint32_t lanes = 4;
  Sampling sampling(V16, lanes);
  hipStream_t stream;
  hip(hipStreamCreate(&stream));
  std::vector<float> logits((size_t)lanes * rows * V16);
  for (uint32_t r = 0; r < lanes * rows; ++r)
    for (uint32_t t = 0; t < V16; ++t) logits[(size_t)r * V16 + t] = logit16(r, t);
  std::vector<float> uniforms(lanes * JF_SAMPLING_UNIFORMS);
  for (uint32_t l = 0; l < lanes; ++l)
    for (uint32_t s = 0; s < JF_SAMPLING_UNIFORMS; ++s)
      uniforms[l * JF_SAMPLING_UNIFORMS + s] = uniform(l, s);
  std::vector<uint32_t> inputs((size_t)lanes * rows);
  for (uint32_t i = 0; i < lanes * rows; ++i) inputs[i] = (i * 7717u + 3u) % V16;
  std::vector<uint32_t> cands((size_t)lanes * (rows - 1) * 16);
  std::vector<float> cprobs(cands.size());
  for (uint32_t l = 0; l < lanes; ++l)
    for (uint32_t r = 0; r + 1 < rows; ++r)
      for (uint32_t j = 0; j < 16; ++j) {
        const size_t k = ((size_t)l * (rows - 1) + r) * 16 + j;
        cands[k] = j ? (r * 5303u + j * 9721u + l) % V16 : inputs[l * rows + r + 1];
        cprobs[k] = j ? 0.01f : 0.6f;
      }
  jf_penalty_table *table = nullptr;
  if (jf_penalty_table_create(V16, lanes, 4096, &table) != JF_OK)
    throw std::runtime_error(jf_last_error());
  // Table row 1 for lane 0, row 3 for lane 2 (lanes 1 and 3 unpenalized).
  for (uint32_t t = 1; t < 4; t += 2) {
    std::vector<uint32_t> history(1500);
    for (uint32_t i = 0; i < history.size(); ++i) history[i] = (i * 131071u + t * 977u) % V16;
    for (uint32_t i = 0; i < 40; ++i) history[1000 + i] = inputs[(t == 1 ? 0 : 2) * rows + 1 + (i % 5)];
    if (jf_penalty_table_rebuild(table, t, history.data(), history.size(), 700, 0, 0, 1,
                                 stream) != JF_OK)
      throw std::runtime_error(jf_last_error());
  }
  const std::vector<uint32_t> stateLanes{1, JF_NO_TOKEN, 3, JF_NO_TOKEN};
  SamplingBuffers b;
  b.logits = upload(logits);
  b.uniforms = upload(uniforms);
  b.inputTokens = upload(inputs);
  b.draftCandidates = upload(cands);
  b.draftProbabilities = upload(cprobs);
  b.outputTokens = upload(std::vector<uint32_t>((size_t)lanes * rows, 0));
  b.targetProbabilities = upload(std::vector<float>((size_t)lanes * rows, 0.0f));
  SamplingPolicy penalized;
  penalized.temperature = 0.9f;
  penalized.topK = 40;
  penalized.topP = 0.92f;
  penalized.penalties.repetition = 1.15f;
  penalized.penalties.presence = 0.4f;
  penalized.penalties.frequency = 0.25f;
  SamplingPolicy plain;
  plain.temperature = 0.7f;
  plain.topK = 20;
  SamplingPolicy greedy;
  const std::vector<SamplingPolicy> policies{penalized, plain, penalized, greedy};
  sampling.addVerify(stream, policies, b, JF_NO_TOKEN, JF_NO_TOKEN,
                     PenaltyTable{table, stateLanes});
  hip(hipStreamSynchronize(stream));
  const std::vector<uint32_t> verifyTokens = download<uint32_t>(b.outputTokens);
  const std::vector<float> verifyProbs = download<float>(b.targetProbabilities);
  AcceptanceBuffers ab;
  std::vector<uint32_t> proposed((size_t)lanes * (rows - 1));
  for (uint32_t l = 0; l < lanes; ++l)
    for (uint32_t r = 0; r + 1 < rows; ++r) proposed[l * (rows - 1) + r] = inputs[l * rows + r + 1];
  ab.proposedTokens = upload(proposed);
  ab.candidates = b.draftCandidates;
  ab.proposalProbabilities = b.draftProbabilities;
  ab.targetProbabilities = b.targetProbabilities;
  ab.uniforms = b.uniforms;
  ab.outputTokens = b.outputTokens;
  ab.retainedCounts = upload(std::vector<uint32_t>(lanes, 0));
  ab.acceptedCounts = upload(std::vector<uint32_t>(lanes, 0));
  const std::vector<uint32_t> maximumRetained{16, 9, 12, 16};
  sampling.addAcceptance(stream, ab, maximumRetained, policies, JF_NO_TOKEN, JF_NO_TOKEN);
  hip(hipStreamSynchronize(stream));
  const std::vector<uint32_t> accepted = download<uint32_t>(ab.outputTokens);
  const std::vector<uint32_t> retained = download<uint32_t>(ab.retainedCounts);
  const std::vector<uint32_t> acceptedCounts = download<uint32_t>(ab.acceptedCounts);
  // The tree form: row r draws its own uniform 24 + r; the first 7 rows
  // carry drafts.
  sampling.addVerify(stream, policies, b, JF_NO_TOKEN, JF_NO_TOKEN,
                     PenaltyTable{table, stateLanes}, true);
  hip(hipStreamSynchronize(stream));
  const std::vector<uint32_t> treeTokens = download<uint32_t>(b.outputTokens);
  const std::vector<float> treeProbs = download<float>(b.targetProbabilities);
  std::printf("{\n");
  print_u32("verify_tokens", verifyTokens);
  print_f32("verify_probs_bits", verifyProbs);
  print_u32("accepted_tokens", accepted);
  print_u32("retained", retained);
  print_u32("accepted", acceptedCounts);
  print_u32("tree_tokens", treeTokens);
  print_f32("tree_probs_bits", treeProbs);
  std::printf("\"gpu_failures\": %d\n}\n", failures);
  jf_penalty_table_destroy(table);
  for (DeviceBuffer *d : {&b.logits, &b.uniforms, &b.inputTokens, &b.draftCandidates,
                          &b.draftProbabilities, &b.outputTokens, &b.targetProbabilities,
                          &ab.proposedTokens, &ab.retainedCounts, &ab.acceptedCounts})
    hip(hipFree(d->data));
  hip(hipStreamDestroy(stream));
  return failures ? 1 : 0;
}

}  // namespace

int main(int argc, char **argv) {
  const std::string mode = argc > 1 ? argv[1] : "cpu";
  try {
    if (mode == "verify16") return gpu_verify16();
    return mode == "gpu" ? gpu_checks() : cpu_checks();
  } catch (const std::exception &e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 2;
  }
}
