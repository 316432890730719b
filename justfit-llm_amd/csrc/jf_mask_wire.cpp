// The mask wire format between the engine's grammar and the runtime
// (source/runtime/engine/Protocol.hpp:22-25, 34-50, 185-203, 263-278;
// Protocol.cpp:195-204, 402-414, 469-500, 616-632, 793-820) and the checks and
// row rules around it (Runtime::provideMask, Runtime.cpp:3449-3483;
// rust/frontend/src/grammar.rs:222-270). A frame is a 16-byte header
// ("SPLH", u16 protocol version 9, u16 frame type, u64 payload bytes) and
// the payload, every integer little-endian. Host code.
#include "jf_sampler.h"

#include "jf_host.h"

#include <cstring>
#include <string>


namespace {

constexpr uint16_t kVersion = 9;
constexpr uint64_t kHeader = 16;
constexpr uint64_t kRequestFixed = 24;   // ids, words per mask, count
constexpr uint64_t kResponseFixed = 20;  // ids, word count
constexpr uint32_t kMaxSimulation = 32;  // ProtocolLimits::maxSimulationTokens
constexpr uint32_t kMaxWords = 1u << 20; // ProtocolLimits::maxMaskWords

void put_le(uint8_t *p, uint64_t v, int bytes) {
  for (int i = 0; i < bytes; ++i) p[i] = (uint8_t)(v >> (8 * i));
}
uint64_t get_le(const uint8_t *p, int bytes) {
  uint64_t v = 0;
  for (int i = 0; i < bytes; ++i) v |= (uint64_t)p[i] << (8 * i);
  return v;
}
int invalid(const char *message) { return jf::set_error(JF_ERR_INVALID_ARGUMENT, message); }

}  // namespace

extern "C" {

int jf_mask_request_encode(uint64_t request_id, uint64_t mask_request_id, uint32_t words_per_mask,
                           const uint32_t *tokens, uint32_t count, const uint32_t *parents,
                           uint8_t *out, uint64_t capacity, uint64_t *written) {
  if (written) *written = 0;
  // validateMaskRequest (Protocol.cpp:469-500).
  if (!request_id || !mask_request_id) return invalid("mask request ids must be non-zero");
  if (!words_per_mask || count > kMaxSimulation || (count && !tokens))
    return invalid("mask request dimensions are invalid");
  if (parents) {
    bool tree = count > 0 && parents[0] == 0;
    for (uint32_t row = 1; tree && row < count; ++row) tree = parents[row] < row;
    if (!tree) return invalid("mask tree parents are invalid");
  }
  if ((uint64_t)words_per_mask * (count + 1u) > kMaxWords)
    return invalid("mask request output would exceed the mask limit");
  const uint64_t payload = kRequestFixed + (uint64_t)count * 4u * (parents ? 2u : 1u);
  if (!out || !written || capacity < kHeader + payload)
    return invalid("mask request output buffer too small");
  std::memcpy(out, "SPLH", 4);
  put_le(out + 4, kVersion, 2);
  put_le(out + 6, parents ? JF_FRAME_MASK_TREE_REQUEST : JF_FRAME_MASK_REQUEST, 2);
  put_le(out + 8, payload, 8);
  uint8_t *p = out + kHeader;
  put_le(p, request_id, 8);
  put_le(p + 8, mask_request_id, 8);
  put_le(p + 16, words_per_mask, 4);
  put_le(p + 20, count, 4);
  for (uint32_t i = 0; i < count; ++i) put_le(p + 24 + 4 * i, tokens[i], 4);
  if (parents)
    for (uint32_t i = 0; i < count; ++i) put_le(p + 24 + 4 * (count + i), parents[i], 4);
  *written = kHeader + payload;
  return JF_OK;
}

int jf_mask_response_decode(const uint8_t *frame, uint64_t bytes, uint64_t *request_id,
                            uint64_t *mask_request_id, uint32_t *words, uint32_t capacity,
                            uint32_t *count) {
  if (!frame || !request_id || !mask_request_id || !count)
    return invalid("mask response arguments are null");
  *count = 0;
  if (bytes < kHeader || std::memcmp(frame, "SPLH", 4) != 0)
    return invalid("frame header is malformed");
  if (get_le(frame + 4, 2) != kVersion) return invalid("frame protocol version is unsupported");
  if (get_le(frame + 6, 2) != JF_FRAME_MASK_RESPONSE) return invalid("frame is not a mask response");
  const uint64_t payload = get_le(frame + 8, 8);
  if (payload != bytes - kHeader) return invalid("frame payload length does not match the frame");
  // decodeMaskResponse (Protocol.cpp:793-820).
  const uint8_t *p = frame + kHeader;
  if (payload < kResponseFixed) return invalid("mask response fixed payload is truncated");
  const uint64_t rid = get_le(p, 8), mid = get_le(p + 8, 8);
  const uint32_t n = (uint32_t)get_le(p + 16, 4);
  if (n > kMaxWords) return invalid("mask response word count exceeds its limit");
  if (payload - kResponseFixed != (uint64_t)n * 4u)
    return invalid("mask word count does not match the binary payload");
  // validateMaskResponse (Protocol.cpp:402-414).
  if (!rid || !mid) return invalid("mask response request ids must be non-zero");
  if (!n) return invalid("mask response word count exceeds its limit");
  if (!words || capacity < n) return invalid("mask response output buffer too small");
  for (uint32_t i = 0; i < n; ++i) words[i] = (uint32_t)get_le(p + kResponseFixed + 4u * i, 4);
  *request_id = rid;
  *mask_request_id = mid;
  *count = n;
  return JF_OK;
}

int jf_mask_rows_check(const uint32_t *words, uint32_t rows, uint32_t mask_words,
                       uint32_t pending_token) {
  if (!words || !rows || !mask_words) return invalid("token mask has the wrong word count");
  // Runtime::provideMask (Runtime.cpp:3466-3481).
  for (uint32_t r = 0; r < rows; ++r) {
    const uint32_t *row = words + (uint64_t)r * mask_words;
    bool any = false;
    for (uint32_t w = 0; w < mask_words && !any; ++w) any = row[w] != 0;
    if (!any) return invalid("token mask row permits no vocabulary token");
  }
  if (pending_token != JF_NO_TOKEN &&
      (pending_token / 32u >= mask_words || !((words[pending_token / 32u] >> (pending_token % 32u)) & 1u)))
    return invalid("verify mask is not synchronized to the pending anchor");
  return JF_OK;
}

int jf_mask_chain_fill(uint32_t *words, uint32_t count, uint32_t valid, uint32_t mask_words) {
  // grammar.rs:255-266: rows 0..valid hold masks; the rest repeat row valid.
  if (!words || !mask_words || valid > count) return invalid("invalid mask chain rows");
  for (uint32_t r = valid + 1; r <= count; ++r)
    std::memcpy(words + (uint64_t)r * mask_words, words + (uint64_t)valid * mask_words,
                mask_words * sizeof(uint32_t));
  return JF_OK;
}

int jf_mask_tree_fill(uint32_t *words, uint32_t count, const uint32_t *parents,
                      const uint8_t *refused, uint32_t mask_words) {
  // grammar.rs:226-250: mask row 0 is the state before the anchor, row
  // r + 1 the state after token row r's path; a token row whose path the
  // grammar refuses (its own token, or an ancestor's) takes the mask of its
  // parent's row (row 0 for the anchor).
  if (!words || !parents || !refused || !count || count > JF_TREE_MAXIMUM_ROWS || !mask_words ||
      parents[0] != 0)
    return invalid("invalid tree mask request");
  for (uint32_t r = 1; r < count; ++r)
    if (parents[r] >= r) return invalid("invalid tree mask request");
  bool dead[JF_TREE_MAXIMUM_ROWS] = {};
  for (uint32_t r = 0; r < count; ++r) {
    dead[r] = refused[r] != 0 || (r > 0 && dead[parents[r]]);
    if (dead[r]) {
      const uint32_t src = r == 0 ? 0u : parents[r] + 1u;
      std::memcpy(words + (uint64_t)(r + 1) * mask_words, words + (uint64_t)src * mask_words,
                  mask_words * sizeof(uint32_t));
    }
  }
  return JF_OK;
}

}  // extern "C"
