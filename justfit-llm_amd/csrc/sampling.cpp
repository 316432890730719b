// justfit::hip::Sampling over the C ABI (see sampling.hpp). The reference's
// row addressing (metal/abi/Sampling.h:31-39) maps onto jf_sample's strides:
// selected row s of lane l reads logits row l * verifyRows + logitsRow + r,
// mask row l * (verifyRows + 1) + maskRow + r and uniform l * 40 + slot.
#include "sampling.hpp"

#include <stdexcept>
#include <string>

namespace justfit::hip {
namespace {

thread_local uint32_t currentVerifyRows = 8;

void check(int rc) {
  if (rc == JF_OK) return;
  const std::string message = jf_last_error();
  if (rc == JF_ERR_INVALID_ARGUMENT) throw std::invalid_argument(message);
  if (rc == JF_ERR_LOGIC) throw std::logic_error(message);
  throw std::runtime_error(message);
}

// BufferExtent.hpp:24-28
void requireBytes(const DeviceBuffer &buffer, uint64_t bytes,
                  const char *what) {
  if (buffer.sizeBytes < bytes)
    throw std::invalid_argument(std::string(what) + " buffer holds " +
                                std::to_string(buffer.sizeBytes) +
                                " bytes, needs " + std::to_string(bytes));
}

jf_policy toPolicy(const SamplingPolicy &p) {
  jf_policy out{};
  out.top_k = p.topK;
  out.temperature = p.temperature;
  out.top_p = p.topP;
  out.min_p = p.minP;
  out.repetition = p.penalties.repetition;
  out.presence = p.penalties.presence;
  out.frequency = p.penalties.frequency;
  out.flags = (p.constrained ? JF_POLICY_CONSTRAINED : 0u) |
              (p.excludesStopTokens ? JF_POLICY_EXCLUDE_STOP : 0u);
  return out;
}

}  // namespace

uint32_t activeVerifyRows() noexcept { return currentVerifyRows; }

VerifyShapeScope::VerifyShapeScope(uint32_t rows) : prior_(currentVerifyRows) {
  if (rows != 8 && rows != 16)
    throw std::invalid_argument("verify shape must be 8 or 16");
  currentVerifyRows = rows;
}
VerifyShapeScope::~VerifyShapeScope() { currentVerifyRows = prior_; }

Sampling::Sampling(uint32_t vocabulary, uint32_t maximumLanes)
    : vocabulary_(vocabulary), maskWords_((vocabulary + 31) / 32),
      maximumLanes_(maximumLanes) {
  if (!vocabulary) throw std::invalid_argument("invalid sampling geometry");
  if (!maximumLanes) throw std::invalid_argument("invalid sampling batch width");
  check(jf_sampler_create(vocabulary, maximumLanes * 16, &sampler_));
  // Row r of lane l draws slot l * 40 + 24 + r (tree) or l * 40 + 15
  // (the correction), Sampling.h:19-29.
  const size_t per = (size_t)maximumLanes * 16;
  std::vector<uint32_t> index(4 * per);
  for (uint32_t t = 0; t < 4; ++t) {
    const bool tree = t & 1u;
    const uint32_t rows = (t & 2u) ? 16u : 8u;
    for (uint32_t l = 0; l < maximumLanes; ++l)
      for (uint32_t r = 0; r < rows; ++r)
        index[t * per + l * rows + r] =
            l * JF_SAMPLING_UNIFORMS + (tree ? JF_UNIFORM_TREE_DRAWS + r : JF_UNIFORM_CORRECTION);
  }
  hipError_t e = hipMalloc((void **)&uniformIndex_, index.size() * sizeof(uint32_t));
  if (e == hipSuccess)
    e = hipMemcpy(uniformIndex_, index.data(), index.size() * sizeof(uint32_t),
                  hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(uniformIndex_);
    jf_sampler_destroy(sampler_);
    throw std::runtime_error(std::string("uniform index table: ") + hipGetErrorString(e));
  }
}

Sampling::~Sampling() {
  (void)hipFree(uniformIndex_);
  jf_sampler_destroy(sampler_);
}

void Sampling::rebuildPenaltyWords(std::span<uint32_t> words,
                                   std::span<const uint32_t> history,
                                   uint64_t generatedTokens,
                                   std::optional<uint32_t> pendingToken,
                                   bool markPrompt) {
  check(jf_penalty_words_rebuild(
      words.data(), (uint32_t)words.size(), history.data(), history.size(),
      generatedTokens, pendingToken.has_value(),
      pendingToken.value_or(0), markPrompt));
}

void Sampling::countPenaltyTokens(std::span<uint32_t> words,
                                  std::span<const uint32_t> selected) {
  check(jf_penalty_words_count(words.data(), (uint32_t)words.size(),
                               selected.data(), selected.size()));
}

// Sampling.cpp:134-147: one row per lane, row rowOffset, uniform 0.
void Sampling::addInitial(hipStream_t stream,
                          std::span<const SamplingPolicy> policies,
                          const SamplingBuffers &buffers, uint32_t rowOffset,
                          uint32_t stopToken0, uint32_t stopToken1,
                          const PenaltyTable &penalties) const {
  if (policies.empty() || policies.size() > maximumLanes_)
    throw std::invalid_argument("invalid sampling batch width");
  const uint32_t rows = activeVerifyRows();
  if (rowOffset >= rows)
    throw std::invalid_argument("invalid initial sampling row");
  const uint64_t lanes = policies.size();
  requireBytes(buffers.logits,
               ((lanes - 1) * rows + rowOffset + 1) * vocabulary_ * sizeof(float),
               "sampling logits");
  requireBytes(buffers.outputTokens, lanes * sizeof(uint32_t), "sampled token");
  std::vector<jf_policy> ps;
  std::vector<uint32_t> penaltyRows;
  bool constrained = false, sampled = false;
  for (uint32_t l = 0; l < lanes; ++l) {
    ps.push_back(toPolicy(policies[l]));
    constrained |= policies[l].constrained;
    sampled |= policies[l].samples();
    penaltyRows.push_back(l < penalties.rows.size() ? penalties.rows[l]
                                                    : JF_NO_TOKEN);
  }
  if (constrained)
    requireBytes(buffers.constraintMasks,
                 ((lanes - 1) * (rows + 1) + 1) * maskWords_ * sizeof(uint32_t),
                 "constraint mask");
  if (sampled)
    requireBytes(buffers.uniforms,
                 ((lanes - 1) * JF_SAMPLING_UNIFORMS + 1) * sizeof(float),
                 "sampling uniform");
  jf_sample_args a{};
  a.rows = (uint32_t)lanes;
  a.dtype = JF_DTYPE_F32;
  a.logits = (const float *)buffers.logits.data + (uint64_t)rowOffset * vocabulary_;
  a.logits_stride = (uint64_t)rows * vocabulary_;
  a.masks = (const uint32_t *)buffers.constraintMasks.data;
  a.mask_stride = (uint64_t)(rows + 1) * maskWords_;
  a.policies = ps.data();
  a.stop_token_0 = stopToken0;
  a.stop_token_1 = stopToken1;
  a.penalties = penalties.words;
  a.penalty_rows = penaltyRows.data();
  a.uniforms = (const float *)buffers.uniforms.data;
  a.uniform_offset = JF_UNIFORM_INITIAL;
  a.uniform_stride = JF_SAMPLING_UNIFORMS;
  a.out_tokens = (uint32_t *)buffers.outputTokens.data;
  check(jf_sample(sampler_, &a, stream));
}

// Sampling.cpp:149-172: every verify row of each lane; row r reads mask row
// r + 1 and follows draft token r (input row r + 1) below the drafted rows;
// rows draw the correction uniform, or their own tree uniform 24 + r.
void Sampling::addVerify(hipStream_t stream,
                         std::span<const SamplingPolicy> policies,
                         const SamplingBuffers &buffers, uint32_t stopToken0,
                         uint32_t stopToken1, const PenaltyTable &penalties,
                         bool tree) const {
  if (policies.empty() || policies.size() > maximumLanes_)
    throw std::invalid_argument("invalid sampling batch width");
  const uint32_t rows = activeVerifyRows();
  const uint32_t drafted = tree ? 7u : rows - 1;
  const uint64_t lanes = policies.size();
  requireBytes(buffers.logits, lanes * rows * vocabulary_ * sizeof(float),
               "sampling logits");
  requireBytes(buffers.outputTokens, lanes * rows * sizeof(uint32_t),
               "sampled token");
  requireBytes(buffers.inputTokens, lanes * rows * sizeof(uint32_t),
               "verify input token");
  requireBytes(buffers.targetProbabilities, lanes * rows * sizeof(float),
               "target probability");
  for (uint32_t l = 0; l < lanes; ++l) {
    const SamplingPolicy &policy = policies[l];
    if (policy.constrained)
      requireBytes(buffers.constraintMasks,
                   (l * (rows + 1) + 1 + rows) * (uint64_t)maskWords_ * sizeof(uint32_t),
                   "constraint mask");
    if (policy.samples()) {
      requireBytes(buffers.uniforms, (uint64_t)(l + 1) * JF_SAMPLING_UNIFORMS * sizeof(float),
                   "sampling uniform");
      requireBytes(buffers.draftCandidates,
                   (l * (rows - 1) + drafted) * (uint64_t)JF_DRAFT_CANDIDATES * sizeof(uint32_t),
                   "draft candidate");
      requireBytes(buffers.draftProbabilities,
                   (l * (rows - 1) + drafted) * (uint64_t)JF_DRAFT_CANDIDATES * sizeof(float),
                   "draft probability");
    }
  }
  // One selection over every row of every lane (the reference's one
  // dispatch set): row g = l * rows + r reads logits row g, mask row
  // l * (rows + 1) + 1 + r, input rows 1..r of its lane as extra penalty
  // tokens, draft token input row r + 1 with candidates l * (rows - 1) + r
  // below the drafted rows, and its lane's correction or tree uniform.
  const uint32_t total = (uint32_t)lanes * rows;
  std::vector<jf_policy> ps(total);
  std::vector<uint32_t> penaltyRows(total), extra(total), maskRows(total),
      draftIndex(total), candIndex(total);
  std::vector<uint64_t> extraOffsets(total);
  for (uint32_t l = 0; l < lanes; ++l) {
    const jf_policy p = toPolicy(policies[l]);
    const uint32_t penaltyRow =
        l < penalties.rows.size() ? penalties.rows[l] : JF_NO_TOKEN;
    for (uint32_t r = 0; r < rows; ++r) {
      const uint32_t g = l * rows + r;
      ps[g] = p;
      penaltyRows[g] = penaltyRow;
      extra[g] = r;
      extraOffsets[g] = (uint64_t)l * rows + 1;
      maskRows[g] = l * (rows + 1) + 1 + r;
      draftIndex[g] = r < drafted ? l * rows + r + 1 : JF_NO_TOKEN;
      candIndex[g] = l * (rows - 1) + r;
    }
  }
  const uint32_t table = (tree ? 1u : 0u) | (rows == 16 ? 2u : 0u);
  jf_sample_args a{};
  a.rows = total;
  a.dtype = JF_DTYPE_F32;
  a.logits = buffers.logits.data;
  a.logits_stride = vocabulary_;
  a.masks = (const uint32_t *)buffers.constraintMasks.data;
  a.mask_stride = maskWords_;
  a.mask_rows = maskRows.data();
  a.policies = ps.data();
  a.stop_token_0 = stopToken0;
  a.stop_token_1 = stopToken1;
  a.penalties = penalties.words;
  a.penalty_rows = penaltyRows.data();
  a.extra_tokens = (const uint32_t *)buffers.inputTokens.data;
  a.extra_counts = extra.data();
  a.extra_offsets = extraOffsets.data();
  a.uniforms = (const float *)buffers.uniforms.data;
  a.uniform_index = uniformIndex_ + (size_t)table * maximumLanes_ * 16;
  a.draft_tokens = (const uint32_t *)buffers.inputTokens.data;
  a.draft_token_index = draftIndex.data();
  a.draft_cand_ids = (const uint32_t *)buffers.draftCandidates.data;
  a.draft_cand_probs = (const float *)buffers.draftProbabilities.data;
  a.draft_cand_index = candIndex.data();
  a.out_tokens = (uint32_t *)buffers.outputTokens.data;
  a.out_draft_probs = (float *)buffers.targetProbabilities.data;
  check(jf_sample(sampler_, &a, stream));
}

// Sampling.cpp:278-328
void Sampling::addAcceptance(hipStream_t stream,
                             const AcceptanceBuffers &buffers,
                             std::span<const uint32_t> maximumRetained,
                             std::span<const SamplingPolicy> policies,
                             uint32_t stopToken0, uint32_t stopToken1) const {
  if (maximumRetained.empty() || maximumRetained.size() != policies.size() ||
      maximumRetained.size() > maximumLanes_)
    throw std::invalid_argument("invalid DFlash acceptance batch");
  const uint32_t rows = activeVerifyRows();
  const uint64_t lanes = maximumRetained.size();
  requireBytes(buffers.proposedTokens, lanes * (rows - 1) * sizeof(uint32_t),
               "proposed token");
  requireBytes(buffers.outputTokens, lanes * rows * sizeof(uint32_t), "target token");
  requireBytes(buffers.retainedCounts, lanes * sizeof(uint32_t), "retained count");
  requireBytes(buffers.acceptedCounts, lanes * sizeof(uint32_t), "accepted count");
  std::vector<jf_policy> ps;
  for (const SamplingPolicy &p : policies) ps.push_back(toPolicy(p));
  jf_accept_chain_args a{};
  a.lanes = (uint32_t)lanes;
  a.verify_rows = rows;
  a.proposed_tokens = (const uint32_t *)buffers.proposedTokens.data;
  a.candidates = (const uint32_t *)buffers.candidates.data;
  a.proposal_probs = (const float *)buffers.proposalProbabilities.data;
  a.target_draft_probs = (const float *)buffers.targetProbabilities.data;
  a.uniforms = (const float *)buffers.uniforms.data;
  a.target_tokens = (uint32_t *)buffers.outputTokens.data;
  a.retained_counts = (uint32_t *)buffers.retainedCounts.data;
  a.accepted_counts = (uint32_t *)buffers.acceptedCounts.data;
  a.maximum_retained = maximumRetained.data();
  a.policies = ps.data();
  a.stop_token_0 = stopToken0;
  a.stop_token_1 = stopToken1;
  check(jf_accept_chain(sampler_, &a, stream));
}

}  // namespace justfit::hip
