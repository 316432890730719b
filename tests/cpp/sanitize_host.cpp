// Host-only code under AddressSanitizer and UndefinedBehaviorSanitizer: the
// library's host sources (jf_host.cpp, jf_tree.cpp, jf_mask_wire.cpp) and
// the CPU oracle (oracle/jf_oracle.c), built with a plain host compiler and
// driven over seeded random and malformed inputs. Besides running clean, it
// checks the penalty table's device updates: each counted token's update,
// applied to a copy of the device arrays the way penalty_count_kernel
// applies it, must leave them equal to a fresh upload of the host rows.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <random>
#include <vector>

#include "jf_host.h"
#include "jf_oracle.h"
#include "jf_sampler.h"

namespace {

int g_failures = 0;

void expect(bool ok, const char *what, long detail = 0) {
  if (!ok) {
    if (g_failures < 20) std::fprintf(stderr, "FAIL: %s (%ld)\n", what, detail);
    ++g_failures;
  }
}

// The device copy of one table row, updated the way penalty_count_kernel
// does it: entries [index, entries) and slots [slot, slot_used) move up one
// place on an insertion, offsets past the token's bucket grow by one.
struct DeviceRow {
  std::vector<jf::PenaltyEntry> entries;
  std::vector<uint32_t> offsets, slots;
};

void apply(DeviceRow &d, const jf::PenaltyOp &op, uint32_t slot_count) {
  if (op.insert) {
    for (uint32_t p = op.entries; p > op.index; --p) d.entries[p] = d.entries[p - 1];
    for (size_t b = op.token / jf::kPenaltyBucket + 1; b < d.offsets.size(); ++b) ++d.offsets[b];
  }
  d.entries[op.index] = jf::PenaltyEntry{op.token, op.word};
  if (op.slot != jf::kNoSlot) {
    uint32_t *sl = d.slots.data() + (size_t)(op.token / jf::kPenaltyChunk) * slot_count;
    if (op.insert)
      for (uint32_t p = op.slot_used; p > op.slot; --p) sl[p] = sl[p - 1];
    sl[op.slot] = op.slot_value;
  }
}

void check_penalty_rows(std::mt19937 &rng) {
  for (uint32_t V : {20000u, 151936u}) {
    const uint32_t rows = 3, max_entries = 1200, slot_count = 256;
    jf::PenaltyRows host;
    host.init(V, rows, max_entries, slot_count);
    for (int trial = 0; trial < 6; ++trial) {
      const uint32_t row = trial % rows;
      // A history clustered in the first chunk half the time, so rows fill
      // one chunk's slots and stop fitting.
      const bool clustered = trial % 2 == 1;
      std::vector<uint32_t> history(300 + rng() % 500);
      for (uint32_t &t : history)
        t = clustered ? rng() % std::min<uint32_t>(V, 600) : rng() % V;
      const uint64_t generated = rng() % history.size();
      std::vector<uint32_t> words(V);
      expect(jf_penalty_words_rebuild(words.data(), V, history.data(), history.size(),
                                      generated, 0, 0, trial % 3 == 0) == JF_OK,
             "rebuild words");
      expect(host.rebuild(row, words.data()) == JF_OK, "rebuild rows");
      DeviceRow d;
      d.entries.assign(max_entries, jf::PenaltyEntry{0, 0});
      host.entries(row, d.entries.data());
      d.offsets.assign(host.buckets() + 1, 0);
      host.offsets(row, d.offsets.data());
      d.slots.assign((size_t)host.chunks() * slot_count, 0);
      host.slots(row, d.slots.data());
      bool slots_kept = host.fits(row);
      std::vector<jf::PenaltyEntry> h;
      for (int k = 0; k < 400; ++k) {
        h.assign(host.size(row), jf::PenaltyEntry{0, 0});
        host.entries(row, h.data());
        uint32_t token;
        const uint32_t pick = rng() % 4;
        if (pick < 2 && !h.empty())
          token = h[rng() % h.size()].token;
        else if (pick == 2)
          token = rng() % std::min<uint32_t>(V, 900);
        else
          token = rng() % V;
        jf::PenaltyOp op{};
        const size_t before = h.size();
        const int rc = host.count(row, token, &op);
        if (rc != JF_OK) {
          expect(before == max_entries, "count fails only on a full row", (long)before);
          continue;
        }
        ++words[token];
        apply(d, op, slot_count);
        if (!host.fits(row)) slots_kept = false;
        expect(op.slot != jf::kNoSlot || !slots_kept, "slot kept while fitting");
        // The updated device copy equals a fresh upload of the host row.
        std::vector<jf::PenaltyEntry> h2(host.size(row));
        host.entries(row, h2.data());
        expect(std::equal(h2.begin(), h2.end(), d.entries.begin(),
                          [](const jf::PenaltyEntry &a, const jf::PenaltyEntry &b) {
                            return a.token == b.token && a.word == b.word;
                          }),
               "entries", k);
        std::vector<uint32_t> off(host.buckets() + 1);
        host.offsets(row, off.data());
        expect(off == d.offsets, "offsets", k);
        if (slots_kept) {
          std::vector<uint32_t> sl((size_t)host.chunks() * slot_count);
          host.slots(row, sl.data());
          expect(sl == d.slots, "slots", k);
        }
        // And the dense words the reference keeps.
        size_t nonzero = 0;
        for (const auto &e : h2) {
          expect(words[e.token] == e.word, "word", e.token);
          ++nonzero;
        }
        size_t dense = 0;
        for (uint32_t w : words) dense += w != 0;
        expect(dense == nonzero, "entry count", (long)dense);
      }
    }
  }
}

// A table widened from 256 to 512 slots a chunk lays every row out as a
// table built at 512 does, and fits exactly the rows that fit 512.
void check_slot_widening(std::mt19937 &rng) {
  const uint32_t V = 151936, rows = 4, max_entries = 2048;
  jf::PenaltyRows narrow, wide;
  narrow.init(V, rows, max_entries, 256);
  wide.init(V, rows, max_entries, 512);
  for (uint32_t row = 0; row < rows; ++row) {
    // Row r holds 150 + 150 r distinct ids in the first chunk: 150, 300,
    // 450, 600 (the last fits neither layout).
    std::vector<uint32_t> words(V, 0);
    for (uint32_t k = 0; k < 150 + 150 * row; ++k) words[k * 13 % 8192] = 1 + rng() % 3;
    for (int k = 0; k < 200; ++k) words[8192 + rng() % (V - 8192)] += 1;
    expect(narrow.rebuild(row, words.data()) == JF_OK, "rebuild narrow");
    expect(wide.rebuild(row, words.data()) == JF_OK, "rebuild wide");
    expect(narrow.fits(row) == (row == 0), "narrow fit", row);
    expect(narrow.fits_at(row, 512) == (row < 3), "fit at 512", row);
  }
  narrow.set_slot_count(512);
  for (uint32_t row = 0; row < rows; ++row) {
    expect(narrow.fits(row) == wide.fits(row), "widened fit", row);
    std::vector<uint32_t> a((size_t)narrow.chunks() * 512), b(a.size());
    narrow.slots(row, a.data());
    wide.slots(row, b.data());
    expect(a == b, "widened slots", row);
  }
}

void check_policies() {
  const float temps[] = {0.0f, 1e-39f, 1.17549435e-38f, 0.7f, INFINITY, NAN, -1.0f};
  const float ps[] = {0.0f, 1e-7f, 0.5f, 1.0f, 1.0000001f, NAN};
  const float pens[] = {0.0f, 1.0f, 2.0f, 2.0000002f, -2.0f, NAN, INFINITY};
  for (float t : temps)
    for (float p : ps)
      for (float m : ps)
        for (float pen : pens) {
          jf_policy a{};
          a.top_k = 5;
          a.temperature = t;
          a.top_p = p;
          a.min_p = m;
          a.repetition = pen == 0.0f ? 1.0f : std::fabs(pen);
          a.presence = pen;
          a.frequency = -pen;
          jfo_policy o{a.top_k, a.temperature, a.top_p, a.min_p, a.repetition,
                       a.presence, a.frequency, 0};
          expect((jf_policy_validate(&a) == JF_OK) == (jfo_policy_valid(&o) == 0),
                 "policy rules agree");
        }
}

void check_mask_wire(std::mt19937 &rng) {
  std::vector<uint8_t> buf(1 << 16);
  for (int trial = 0; trial < 300; ++trial) {
    const uint32_t count = rng() % 20;
    std::vector<uint32_t> tokens(count + 1), parents(count + 1);
    for (uint32_t i = 0; i <= count; ++i) {
      tokens[i] = rng();
      parents[i] = i ? rng() % i : 0;
    }
    const bool tree = trial % 2;
    uint64_t written = 0;
    const uint64_t cap = rng() % 3 == 0 ? rng() % 200 : buf.size();
    (void)jf_mask_request_encode(rng(), rng(), 1 + rng() % 8000, tokens.data(), count,
                                 tree ? parents.data() : nullptr, buf.data(), cap, &written);
    // A response frame: valid most of the time, then cut or corrupted.
    const uint32_t words = rng() % 64;
    std::vector<uint8_t> f(16 + 24 + 4 * (size_t)words);
    std::memcpy(f.data(), "SPLH", 4);
    f[4] = 9;
    f[6] = 0x03;
    const uint64_t payload = f.size() - 16;
    for (int i = 0; i < 8; ++i) f[8 + i] = (uint8_t)(payload >> (8 * i));
    for (size_t i = 16; i < f.size(); ++i) f[i] = (uint8_t)rng();
    f[16 + 16] = (uint8_t)words;  // a plausible word count
    f[16 + 17] = f[16 + 18] = f[16 + 19] = 0;
    if (trial % 3 == 1) f[rng() % f.size()] ^= (uint8_t)(1u << (rng() % 8));
    const uint64_t bytes = trial % 3 == 2 ? rng() % f.size() : f.size();
    std::vector<uint32_t> out(64);
    uint64_t rid = 0, mid = 0;
    uint32_t got = 0;
    (void)jf_mask_response_decode(f.data(), bytes, &rid, &mid, out.data(),
                                  (uint32_t)out.size(), &got);
    // Row checks and fills on random masks.
    const uint32_t mw = 1 + rng() % 8, rows = 1 + rng() % 9;
    std::vector<uint32_t> m((size_t)(rows + 1) * mw);
    for (uint32_t &x : m) x = rng() % 4 ? rng() : 0u;
    (void)jf_mask_rows_check(m.data(), rows, mw, rng() % 2 ? rng() % (mw * 32) : JF_NO_TOKEN);
    (void)jf_mask_chain_fill(m.data(), rows, rng() % (rows + 1), mw);
    std::vector<uint8_t> refused(rows + 1);
    for (uint8_t &r : refused) r = rng() % 2;
    std::vector<uint32_t> tree_parents(rows + 1);
    for (uint32_t i = 1; i <= rows; ++i) tree_parents[i] = rng() % 5 ? rng() % i : i + 3;
    (void)jf_mask_tree_fill(m.data(), rows, tree_parents.data(), refused.data(), mw);
  }
}

void check_tree_builder(std::mt19937 &rng) {
  std::uniform_real_distribution<float> U(-8.0f, 8.0f);
  for (int trial = 0; trial < 200; ++trial) {
    std::vector<uint32_t> cand(7 * 16);
    std::vector<float> unary(7 * 16), edges(7 * 16 * 16);
    for (uint32_t &c : cand) c = rng() % 1000;
    for (float &u : unary) u = trial % 7 == 0 ? std::round(U(rng)) : U(rng);
    for (float &e : edges) e = U(rng);
    uint32_t picks[7];
    for (uint32_t &p : picks) p = rng() % 16;
    const uint32_t rows = 1 + rng() % 16;
    jf_draft_tree t{};
    double expected = 0, chain = 0;
    const int rc = jf_build_draft_tree(cand.data(), unary.data(), edges.data(), rng() % 1000,
                                       rows, trial % 2 ? picks : nullptr, &t, &expected, &chain);
    expect(rc == JF_OK, "tree builder");
    if (rc != JF_OK) continue;
    expect(t.rows >= 1 && t.rows <= rows, "tree rows", t.rows);
    for (uint32_t r = 1; r < t.rows; ++r) expect(t.parent[r] < r, "parent order", r);
  }
  jf_draft_tree t{};
  expect(jf_build_draft_tree(nullptr, nullptr, nullptr, 0, 4, nullptr, &t, nullptr, nullptr) !=
             JF_OK,
         "tree builder rejects null inputs");
}

uint16_t bf16_of(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  return (uint16_t)(u >> 16);
}

void check_oracle(std::mt19937 &rng) {
  std::normal_distribution<float> N(0.0f, 3.0f);
  std::uniform_real_distribution<float> U01(0.0f, 1.0f);
  for (int trial = 0; trial < 400; ++trial) {
    const uint32_t V = 1 + rng() % 400;
    std::vector<float> lg(V);
    std::vector<uint16_t> lb(V);
    for (uint32_t i = 0; i < V; ++i) {
      const uint32_t r = rng() % 50;
      lg[i] = r == 0 ? NAN : r == 1 ? INFINITY : r == 2 ? -INFINITY : N(rng);
      lb[i] = bf16_of(lg[i]);
    }
    std::vector<uint32_t> mask((V + 31) / 32), words(V);
    for (uint32_t &m : mask) m = rng();
    for (uint32_t &w : words) w = rng() % 5 == 0 ? (rng() % 3) | (rng() % 2 ? 0x80000000u : 0u) : 0u;
    std::vector<uint32_t> extra(rng() % 5), cid(16);
    for (uint32_t &e : extra) e = rng() % V;
    std::vector<float> cpr(16), dq(V);
    for (uint32_t j = 0; j < 16; ++j) {
      cid[j] = rng() % V;
      cpr[j] = U01(rng);
    }
    for (float &q : dq) q = U01(rng) / V;
    jfo_policy p{};
    p.top_k = rng() % 3 ? rng() % (V + 3) : 0;
    p.temperature = rng() % 4 ? 0.05f + 2.0f * U01(rng) : 0.0f;
    p.top_p = rng() % 2 ? 0.05f + 0.95f * U01(rng) : 1.0f;
    p.min_p = rng() % 2 ? 0.3f * U01(rng) : 0.0f;
    p.repetition = rng() % 2 ? 0.5f + U01(rng) : 1.0f;
    p.presence = rng() % 2 ? 2.0f * U01(rng) - 1.0f : 0.0f;
    p.frequency = rng() % 2 ? 2.0f * U01(rng) - 1.0f : 0.0f;
    p.flags = (rng() % 3 == 0 ? JFO_ROW_CONSTRAINED : 0u) | (rng() % 3 == 0 ? JFO_ROW_EXCLUDE_STOP : 0u);
    jfo_row_input in{};
    const bool bf = trial % 2;
    in.logits = bf ? nullptr : lg.data();
    in.logits_bf16 = bf ? lb.data() : nullptr;
    in.mask = mask.data();
    in.words = rng() % 2 ? words.data() : nullptr;
    in.extra = extra.data();
    in.extra_count = (uint32_t)extra.size();
    in.uniform = U01(rng);
    in.draft_token = rng() % 2 ? rng() % V : JFO_NO_TOKEN;
    if (rng() % 2) {
      in.cand_ids = cid.data();
      in.cand_probs = cpr.data();
    } else {
      in.dense_q = dq.data();
    }
    const uint32_t cap = rng() % 3 ? 0 : 1 + rng() % 64;
    std::vector<uint32_t> kid(cap + 1);
    std::vector<float> kpr(cap + 1);
    jfo_row_output out{};
    const int rc = jfo_select_row(V, rng() % V, JFO_NO_TOKEN, &p, &in, &out,
                                  cap ? kid.data() : nullptr, cap ? kpr.data() : nullptr, cap);
    expect(rc == 0 || jfo_policy_valid(&p) != 0, "oracle select", trial);
    if (rc == 0) expect(out.token < V || out.token == JFO_NO_TOKEN, "oracle token", out.token);
  }
  // Chain and tree acceptance on random lanes.
  for (int trial = 0; trial < 300; ++trial) {
    float u[40], tp[16], cpr[16 * 16];
    uint32_t draft[16], cid[16 * 16], tokens[16], retained = 0, accepted = 0, path[16];
    for (float &x : u) x = U01(rng);
    for (float &x : tp) x = U01(rng);
    for (float &x : cpr) x = U01(rng);
    for (uint32_t &x : draft) x = rng() % 50;
    for (uint32_t &x : cid) x = rng() % 50;
    for (uint32_t &x : tokens) x = rng() % 50;
    jfo_chain_params c{};
    c.proposals = trial % 2 ? 7 : 15;
    c.remaining = 1 + rng() % (c.proposals + 1);
    c.stop0 = rng() % 60;
    c.stop1 = JFO_NO_TOKEN;
    c.sampled = trial % 3 != 0;
    jfo_accept_chain(&c, draft, cid, cpr, tp, u, tokens, &retained, &accepted);
    expect(retained >= 1 && retained <= c.remaining, "chain retained", retained);
    jfo_tree_params t{};
    t.rows = 1 + rng() % 16;
    t.chain_rows = 1 + rng() % t.rows;
    t.remaining = 1 + rng() % 8;
    t.stop0 = t.stop1 = JFO_NO_TOKEN;
    t.sampled = trial % 2;
    for (uint32_t r = 0; r < 16; ++r) {
      t.parent[r] = r ? rng() % r : 0;
      t.token[r] = rng() % 50;
    }
    for (uint32_t r = 1; r < t.chain_rows; ++r) t.parent[r] = r - 1;
    for (float &q : t.chain_q) q = U01(rng);
    jfo_accept_tree(&t, tp, u, tokens, &retained, &accepted, path);
    expect(retained >= 1 && retained <= t.remaining, "tree retained", retained);
  }
  // Draft selector pieces.
  for (int trial = 0; trial < 20; ++trial) {
    const uint32_t V = 16 + rng() % 3000;
    std::vector<float> logits(8 * (size_t)V);
    for (float &x : logits) x = rng() % 97 == 0 ? NAN : N(rng);
    uint32_t ids[16];
    float vals[16];
    jfo_draft_top16(logits.data(), V, ids, vals);
    std::vector<uint16_t> hidden(8 * 256), pred(64 * 256), succ(64 * 256);
    for (uint16_t &h : hidden) h = bf16_of(N(rng) * 0.1f);
    for (uint16_t &h : pred) h = bf16_of(N(rng) * 0.1f);
    for (uint16_t &h : succ) h = bf16_of(N(rng) * 0.1f);
    (void)jfo_draft_edge(pred.data(), hidden.data(), succ.data());
  }
  // Tree gather over a small buffer.
  for (int trial = 0; trial < 50; ++trial) {
    jfo_gather_params g{};
    g.columns = 1 + rng() % 8;
    g.inner = 1 + rng() % g.columns;
    g.inner_stride = 1;
    g.outer_stride = g.inner;
    g.row_stride = g.columns + rng() % 3;
    g.rows = 1 + rng() % 16;
    g.lane_stride = g.row_stride * g.rows;
    g.lanes = 1 + rng() % 3;
    g.layer_stride = g.lane_stride * g.lanes;
    g.layers = 1 + rng() % 2;
    std::vector<uint16_t> data((size_t)g.layer_stride * g.layers);
    for (uint16_t &x : data) x = (uint16_t)rng();
    std::vector<uint32_t> path(8 * g.lanes), retained(g.lanes);
    for (uint32_t &p : path) p = rng() % (g.rows + 2);
    for (uint32_t &r : retained) r = rng() % (std::min<uint32_t>(8, g.rows) + 1);
    jfo_tree_gather(data.data(), path.data(), retained.data(), &g);
  }
}

}  // namespace

int main() {
  std::mt19937 rng(20260);
  check_penalty_rows(rng);
  check_slot_widening(rng);
  check_policies();
  check_mask_wire(rng);
  check_tree_builder(rng);
  check_oracle(rng);
  if (g_failures) {
    std::fprintf(stderr, "%d failures\n", g_failures);
    return 1;
  }
  std::printf("sanitized host checks passed\n");
  return 0;
}
