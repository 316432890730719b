// The draft tree builder (the reference's buildDraftTree,
// source/runtime/model/Runtime.cpp:58-174): one lane's tree from the draft
// selector's candidates, unary scores and edge tables. Nodes are taken best
// first by path log-probability, each node's children scored by a
// log-softmax over its 16 candidates; rows are the DFS preorder with the
// chain first and then children best first; each root-to-leaf path is a
// copy, and each row belongs to the first copy (in DFS order) that holds it.
// Host code; all arithmetic in double as the reference does.
#include "jf_sampler.h"

#include "jf_host.h"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <limits>
#include <queue>
#include <vector>

namespace {

constexpr uint32_t kCands = JF_DRAFT_CANDIDATES;
constexpr uint32_t kPositions = JF_DRAFT_POSITIONS;

struct TreeNode {
  uint32_t token, depth, pick;
  uint32_t parent;  // node index; the anchor's is itself
  double logp;
  bool chain;
  std::vector<uint32_t> children;
};

// A child waiting to be taken: its path log-probability, position, the
// candidate it picks and its parent node.
struct Pending {
  double logp;
  uint32_t position, pick, parent;
};
// "a ranks below b": lower log-probability, then the larger pick. The
// frontier is a binary heap under this order, so equal (logp, pick) pairs
// leave it in the order the reference's std::priority_queue gives them.
struct RanksBelow {
  bool operator()(const Pending &a, const Pending &b) const {
    return a.logp < b.logp || (a.logp == b.logp && a.pick > b.pick);
  }
};

class TreeBuilder {
 public:
  TreeBuilder(const uint32_t *candidates, const float *unary, const float *edges)
      : candidates_(candidates), unary_(unary), edges_(edges) {}

  // Candidate j's score at `position` after predecessor candidate `pred`.
  double score(uint32_t position, uint32_t pred, uint32_t j) const {
    return double(unary_[position * kCands + j]) +
           double(edges_[(position * kCands + pred) * kCands + j]);
  }
  // log sum_j exp(score_j) at (position, pred), as max + log(sum exp(s - max)).
  double normalizer(uint32_t position, uint32_t pred) const {
    double top = -std::numeric_limits<double>::infinity();
    for (uint32_t j = 0; j < kCands; ++j) top = std::max(top, score(position, pred, j));
    double total = 0;
    for (uint32_t j = 0; j < kCands; ++j) total += std::exp(score(position, pred, j) - top);
    return top + std::log(total);
  }
  void expand(uint32_t parent, uint32_t position, uint32_t pred, double base,
              uint32_t skip = UINT32_MAX) {
    const double norm = normalizer(position, pred);
    for (uint32_t j = 0; j < kCands; ++j)
      if (j != skip) frontier_.push({base + score(position, pred, j) - norm, position, j, parent});
  }

  std::vector<TreeNode> build(uint32_t anchor, uint32_t rows, const uint32_t *chain_picks) {
    std::vector<TreeNode> nodes;
    nodes.push_back({anchor, 0, 0, 0, 0.0, chain_picks != nullptr, {}});
    if (chain_picks) {
      // The sampled chain is the leftmost path whatever its scores; the rest
      // are taken best first among its nodes' other children.
      uint32_t parent = 0, pred = 0;
      double logp = 0;
      for (uint32_t position = 0; position < kPositions && nodes.size() < rows; ++position) {
        const uint32_t pick = chain_picks[position];
        const double base = logp;
        logp += score(position, pred, pick) - normalizer(position, pred);
        expand(parent, position, pred, base, pick);
        const uint32_t index = (uint32_t)nodes.size();
        nodes.push_back({candidates_[position * kCands + pick], position + 1, pick, parent, logp,
                         true, {}});
        nodes[parent].children.push_back(index);
        parent = index;
        pred = pick;
      }
    } else {
      expand(0, 0, 0, 0.0);
    }
    while (nodes.size() < rows && !frontier_.empty()) {
      const Pending item = frontier_.top();
      frontier_.pop();
      const uint32_t index = (uint32_t)nodes.size();
      nodes.push_back({candidates_[item.position * kCands + item.pick], item.position + 1,
                       item.pick, item.parent, item.logp, false, {}});
      nodes[item.parent].children.push_back(index);
      if (item.position + 1 < kPositions) expand(index, item.position + 1, item.pick, item.logp);
    }
    return nodes;
  }

  // The selector's own chain (each position's best candidate after the one
  // before): the sum over positions of its cumulative probability.
  double chain_expected() const {
    double total = 0, logp = 0;
    uint32_t pred = 0;
    for (uint32_t position = 0; position < kPositions; ++position) {
      double top = -std::numeric_limits<double>::infinity();
      uint32_t best = 0;
      for (uint32_t j = 0; j < kCands; ++j) {
        const double s = score(position, pred, j);
        if (s > top) {
          top = s;
          best = j;
        }
      }
      double sum = 0;
      for (uint32_t j = 0; j < kCands; ++j) sum += std::exp(score(position, pred, j) - top);
      logp -= std::log(sum);
      total += std::exp(logp);
      pred = best;
    }
    return total;
  }

 private:
  const uint32_t *candidates_;
  const float *unary_;
  const float *edges_;
  std::priority_queue<Pending, std::vector<Pending>, RanksBelow> frontier_;
};

// DFS preorder layout: children with the chain first, then by log-probability
// (larger first), then by pick (smaller first).
void layout(const std::vector<TreeNode> &nodes, jf_draft_tree *tree) {
  std::memset(tree, 0, sizeof(*tree));
  tree->rows = (uint32_t)nodes.size();
  uint32_t next = 0;
  std::vector<uint32_t> stack;
  std::array<bool, JF_TREE_MAXIMUM_ROWS> assigned{};
  auto visit = [&](auto &&self, uint32_t node, uint32_t parent_row) -> void {
    const uint32_t row = next++;
    tree->parent[row] = parent_row;
    tree->depth[row] = nodes[node].depth;
    tree->token[row] = nodes[node].token;
    stack.push_back(row);
    std::vector<uint32_t> children = nodes[node].children;
    std::sort(children.begin(), children.end(), [&](uint32_t a, uint32_t b) {
      if (nodes[a].chain != nodes[b].chain) return nodes[a].chain;
      return nodes[a].logp > nodes[b].logp ||
             (nodes[a].logp == nodes[b].logp && nodes[a].pick < nodes[b].pick);
    });
    if (children.empty()) {
      const uint32_t copy = tree->copies++;
      tree->path_length[copy] = (uint32_t)stack.size();
      for (uint32_t i = 0; i < stack.size(); ++i) tree->path[copy][i] = stack[i];
      for (uint32_t r : stack)
        if (!assigned[r]) {
          assigned[r] = true;
          tree->copy[r] = copy;
        }
    }
    for (uint32_t child : children) self(self, child, row);
    stack.pop_back();
  };
  visit(visit, 0, 0);
}

}  // namespace


extern "C" int jf_build_draft_tree(const uint32_t *candidates, const float *unary,
                                   const float *edges, uint32_t anchor, uint32_t rows,
                                   const uint32_t *chain_picks, jf_draft_tree *out,
                                   double *expected, double *chain_expected) {
  if (!candidates || !unary || !edges || !out || !rows || rows > JF_TREE_MAXIMUM_ROWS)
    return jf::set_error(JF_ERR_INVALID_ARGUMENT, "invalid draft tree arguments");
  if (chain_picks)
    for (uint32_t p = 0; p < kPositions; ++p)
      if (chain_picks[p] >= kCands)
        return jf::set_error(JF_ERR_INVALID_ARGUMENT, "invalid draft chain pick");
  TreeBuilder b(candidates, unary, edges);
  const std::vector<TreeNode> nodes = b.build(anchor, rows, chain_picks);
  layout(nodes, out);
  if (expected) {
    *expected = 0;
    for (size_t i = 1; i < nodes.size(); ++i) *expected += std::exp(nodes[i].logp);
  }
  if (chain_expected) *chain_expected = b.chain_expected();
  return JF_OK;
}
