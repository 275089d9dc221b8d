// rewriter.cpp -- which HLO fragments become ANNC fusions and custom calls.
//
// Host-side restatement of ANNC's KDnnRewriter selection
// (annc/service/cpu/kdnn_rewriter.h:25-59, kdnn_rewriter.cc:8-69), of the
// GEMM patterns (gemm_rewriter.cc:13-134) and of the graph-opt patterns
// (graph_opt.cc:8-50, 52-129), driven by the same ANNC_FLAGS set.  The caller
// describes a fragment as a node array (annc_hlo_node); for one instruction
// the visitor's rewriters are tried by descending benefit and the first that
// matches is reported with its fused nodes and call operands.
//
// Rewriters per visited opcode (kdnn_rewriter.h:98-132):
//   kDot          graph-opt + GEMM rewriters
//   kMultiply     graph-opt rewriters
//   kSelect       graph-opt rewriters
//   kReduceWindow reduce rewriters (none is registered: reduce_rewriter.cc:24-29)
// Benefits: sps-emd-2 3, pooling 3, matmul-add-relu 3, matmul-add 2,
// layout-matmul / matmul / batch-matmul 1.  The reference orders ties with
// std::sort (unspecified); this restatement keeps registration order
// (graph-opt before GEMM; layout-matmul, matmul, batch-matmul).
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "annc_hip.h"
#include "common.h"

namespace annc {
namespace {

struct Graph {
  const annc_hlo_node* nodes;
  int64_t n;
  std::vector<std::vector<int32_t>> users;  // in node-index order

  const annc_hlo_node& at(int32_t i) const { return nodes[i]; }
  // operand k of node i; -1 when node i or its operand k does not exist
  int32_t operand(int32_t i, int k) const {
    return (i >= 0 && k < nodes[i].num_operands) ? nodes[i].operands[k] : -1;
  }
};

// LayoutUtil::IsMonotonicWithDim0Major: minor_to_major is rank-1, ..., 0.
bool dim0_major(const annc_hlo_node& node) {
  for (int d = 0; d < node.rank; ++d)
    if (node.minor_to_major[d] != node.rank - 1 - d) return false;
  return true;
}

struct Pattern {
  int32_t opcode;
  std::vector<int32_t> dtypes;  // per checked operand
  std::vector<int32_t> ranks;   // per checked operand (RewritePattern::dims)
  std::vector<int64_t> min_dims, max_dims;  // on the instruction's shape (dim_range)
  std::vector<Pattern> next;    // users()[i] must match next[i]
};

// match_op_pattern (kdnn_rewriter.cc:8-42); fused nodes are appended in the
// reference's post-order (users first, so the fusion root comes first).
bool match_pattern(const Graph& g, int32_t instr, const Pattern& p, std::vector<int32_t>& fused) {
  const annc_hlo_node& node = g.at(instr);
  if (node.opcode != p.opcode) return false;
  if (node.num_operands < static_cast<int32_t>(p.ranks.size())) return false;
  for (size_t i = 0; i < p.ranks.size(); ++i) {
    const int32_t o = node.operands[i];
    if (o < 0) return false;
    const annc_hlo_node& op = g.at(o);
    if (!dim0_major(op) || op.rank != p.ranks[i] || op.dtype != p.dtypes[i]) return false;
  }
  if (!p.min_dims.empty()) {
    for (int d = 0; d < node.rank; ++d)
      if (node.dims[d] < p.min_dims[d] || node.dims[d] > p.max_dims[d]) return false;
  }
  const std::vector<int32_t>& users = g.users[instr];
  if (users.size() < p.next.size()) return false;
  for (size_t i = 0; i < p.next.size(); ++i)
    if (!match_pattern(g, users[i], p.next[i], fused)) return false;
  fused.push_back(instr);
  return true;
}

// Operands of the fusion XLA builds from `fused` (root first): fusing an
// instruction replaces the parameter that stood for it and appends its
// operands that are not parameters yet (HloFusionInstruction fuse order).
std::vector<int32_t> fusion_operands(const Graph& g, const std::vector<int32_t>& fused) {
  std::vector<int32_t> params;
  for (int32_t instr : fused) {
    auto it = std::find(params.begin(), params.end(), instr);
    if (it != params.end()) params.erase(it);
    const annc_hlo_node& node = g.at(instr);
    for (int k = 0; k < node.num_operands; ++k) {
      const int32_t o = node.operands[k];
      if (o < 0) continue;
      // an operand fused earlier stays inside the fusion
      if (std::find(fused.begin(), fused.end(), o) != fused.end() &&
          std::find(fused.begin(), fused.end(), o) < std::find(fused.begin(), fused.end(), instr))
        continue;
      if (std::find(params.begin(), params.end(), o) == params.end()) params.push_back(o);
    }
  }
  return params;
}

struct Result {
  std::string target;
  bool custom_call = false;
  int benefit = 0;
  std::vector<int32_t> fused;
  std::vector<int32_t> operands;     // -1 / -2: slice starts / limits constants
  std::vector<int32_t> shape_infos;  // node whose get_param_info follows
};

using CustomMatch = bool (*)(const Graph&, int32_t, Result&);

struct Rewriter {
  const char* name;
  int benefit;
  bool dnn_custom_call;  // RewriterType::DNN_CUSTOM_CALL
  CustomMatch custom;    // RewritePattern::custom_rewriter
  Pattern pattern;
};

// match_layout_matmul (gemm_rewriter.cc:13-56): rhs an HLO parameter, both
// operands rank 2 with every dimension >= 12; rhs_format is not consulted.
bool match_layout_matmul(const Graph& g, int32_t dot, Result& r) {
  const annc_hlo_node& node = g.at(dot);
  if (node.opcode != ANNC_HLO_DOT || node.num_operands < 2) return false;
  const int32_t lhs = node.operands[0], rhs = node.operands[1];
  if (lhs < 0 || rhs < 0 || g.at(rhs).opcode != ANNC_HLO_PARAMETER) return false;
  if (g.at(lhs).rank != 2 || g.at(rhs).rank != 2) return false;
  for (int d = 0; d < 2; ++d)
    if (g.at(lhs).dims[d] < 12 || g.at(rhs).dims[d] < 12) return false;
  r.target = "__layout_matmul";
  r.custom_call = true;
  r.fused = {dot};
  const std::vector<int32_t> ops = fusion_operands(g, r.fused);
  r.operands = {ops[0], rhs};
  r.shape_infos = {ops[0], rhs};
  return true;
}

// fused_sparse_embedding2 (graph_opt.cc:8-41): the masked-gather tree under
// a multiply becomes one kLoop fusion (no custom call).
bool match_sparse_embedding2(const Graph& g, int32_t mul, Result& r) {
  auto op = [&](int32_t i, int k) { return g.operand(i, k); };
  auto is = [&](int32_t i, int32_t opc) { return i >= 0 && g.at(i).opcode == opc; };
  if (!is(mul, ANNC_HLO_MULTIPLY)) return false;
  const int32_t broadcast = op(mul, 0), gather = op(mul, 1);
  if (!is(broadcast, ANNC_HLO_BROADCAST) || !is(gather, ANNC_HLO_GATHER)) return false;
  const int32_t select = op(gather, 1);
  if (!is(select, ANNC_HLO_SELECT)) return false;
  const int32_t convert = op(broadcast, 0);
  if (!is(convert, ANNC_HLO_CONVERT)) return false;
  const int32_t and_op = op(convert, 0);
  if (!is(and_op, ANNC_HLO_AND)) return false;
  const int32_t comp0 = op(and_op, 0), comp1 = op(and_op, 1);
  if (!is(comp0, ANNC_HLO_COMPARE) || !is(comp1, ANNC_HLO_COMPARE)) return false;
  if (!is(op(comp1, 0), ANNC_HLO_CONVERT) || !is(op(comp1, 1), ANNC_HLO_BROADCAST)) return false;
  const int32_t broadcast1 = op(comp1, 1);
  if (!is(op(broadcast1, 0), ANNC_HLO_CONSTANT)) return false;
  const int32_t constant1 = op(broadcast1, 0);
  const int32_t broadcast0 = op(comp0, 1);
  if (!is(op(broadcast0, 0), ANNC_HLO_CONSTANT)) return false;
  const int32_t constant0 = op(broadcast0, 0);
  r.target = "sparse_embedding2";
  r.custom_call = false;
  r.fused = {mul, broadcast, gather, select, convert, and_op,
             comp0, comp1, broadcast1, constant1, broadcast0, constant0};
  r.operands = fusion_operands(g, r.fused);
  return true;
}

// fused_pooling (graph_opt.cc:52-118): the masked mean over a padded bag
// becomes the __pooling custom call with operands {fusion operand 5,
// fusion operand 3, slice starts, slice limits, shape(op 5), shape(op 3)}.
bool match_pooling(const Graph& g, int32_t sel, Result& r) {
  auto op = [&](int32_t i, int k) { return g.operand(i, k); };
  auto is = [&](int32_t i, int32_t opc) { return i >= 0 && g.at(i).opcode == opc; };
  if (!is(sel, ANNC_HLO_SELECT)) return false;
  const int32_t broadcast0 = op(sel, 0), divide = op(sel, 2);
  if (!is(broadcast0, ANNC_HLO_BROADCAST) || !is(op(sel, 1), ANNC_HLO_BROADCAST) ||
      !is(divide, ANNC_HLO_DIVIDE))
    return false;
  const int32_t reshape = op(divide, 0), broadcast1 = op(divide, 1);
  if (!is(reshape, ANNC_HLO_RESHAPE) || !is(broadcast1, ANNC_HLO_BROADCAST)) return false;
  const int32_t reduce = op(reshape, 0);
  if (!is(reduce, ANNC_HLO_REDUCE)) return false;
  const int32_t select1 = op(reduce, 0);
  if (!is(select1, ANNC_HLO_SELECT)) return false;
  const int32_t broadcast2 = op(select1, 0), slice = op(select1, 1);
  if (!is(broadcast2, ANNC_HLO_BROADCAST) || !is(slice, ANNC_HLO_SLICE) ||
      !is(op(select1, 2), ANNC_HLO_BROADCAST))
    return false;
  const int32_t compare0 = op(broadcast2, 0);
  if (!is(compare0, ANNC_HLO_COMPARE)) return false;
  const int32_t compare2 = op(broadcast0, 0);
  if (!is(compare2, ANNC_HLO_COMPARE)) return false;
  const int32_t reduce1 = op(compare2, 0);
  if (!is(reduce1, ANNC_HLO_REDUCE)) return false;
  const int32_t convert = op(reduce1, 0);
  if (!is(convert, ANNC_HLO_CONVERT)) return false;
  if (!is(op(convert, 0), ANNC_HLO_COMPARE)) return false;
  r.fused = {sel,        divide,     broadcast1, reshape,  reduce,  select1, slice,
             broadcast2, broadcast0, compare2,   reduce1,  convert, compare0};
  const std::vector<int32_t> ops = fusion_operands(g, r.fused);
  if (ops.size() < 6) return false;
  r.target = "__pooling";
  r.custom_call = true;
  r.operands = {ops[5], ops[3], -1, -2};
  r.shape_infos = {ops[5], ops[3]};
  return true;
}

Pattern gemm_pattern(int rank) {
  Pattern p;
  p.opcode = ANNC_HLO_DOT;
  p.dtypes = {ANNC_DT_F32, ANNC_DT_F32};
  p.ranks = {rank, rank};
  return p;
}

// register_* of gemm_rewriter.cc:65-134 and graph_opt.cc:42-129 for one
// visited instruction, sorted by descending benefit (stable).
std::vector<Rewriter> rewriters_for(int32_t opcode) {
  std::vector<Rewriter> rw;
  const bool dot = opcode == ANNC_HLO_DOT;
  if (dot || opcode == ANNC_HLO_MULTIPLY || opcode == ANNC_HLO_SELECT) {
    if (annc_flag_enabled("sps-emd-2"))
      rw.push_back({"sparse_embedding2", 3, false, match_sparse_embedding2, {}});
    if (annc_flag_enabled("pooling")) rw.push_back({"pooling", 3, false, match_pooling, {}});
  }
  if (dot) {
    if (annc_flag_enabled("layout-matmul"))
      rw.push_back({"layout_matmul", 1, false, match_layout_matmul, {}});
    if (annc_flag_enabled("matmul")) {
      Pattern p = gemm_pattern(2);
      p.min_dims = {12, 12};
      p.max_dims = {INT64_MAX, INT64_MAX};
      rw.push_back({"__matmul", 1, true, nullptr, p});
    }
    if (annc_flag_enabled("batch-matmul")) {
      Pattern p = gemm_pattern(3);
      p.min_dims = {1, 8, 8};
      p.max_dims = {INT64_MAX, INT64_MAX, INT64_MAX};
      rw.push_back({"__batch_matmul", 1, true, nullptr, p});
    }
    if (annc_flag_enabled("matmul-add")) {
      Pattern p = gemm_pattern(2);
      Pattern add;
      add.opcode = ANNC_HLO_ADD;
      p.next = {add};
      rw.push_back({"__matmul_add", 2, true, nullptr, p});
    }
    if (annc_flag_enabled("matmul-add-relu")) {
      Pattern p = gemm_pattern(2);
      Pattern add, mx;
      add.opcode = ANNC_HLO_ADD;
      mx.opcode = ANNC_HLO_MAXIMUM;
      add.next = {mx};
      p.next = {add};
      rw.push_back({"__matmul_add_relu", 3, true, nullptr, p});
    }
  }
  std::stable_sort(rw.begin(), rw.end(),
                   [](const Rewriter& a, const Rewriter& b) { return a.benefit > b.benefit; });
  return rw;
}

}  // namespace
}  // namespace annc

extern "C" int annc_hlo_rewrite_instruction(const annc_hlo_node* nodes, int64_t num_nodes,
                                            int32_t instr, annc_hlo_rewrite* out) {
  using namespace annc;
  ANNC_REQUIRE(nodes && out && num_nodes > 0, "null or empty fragment");
  ANNC_REQUIRE(instr >= 0 && instr < num_nodes, "instruction index out of range");
  for (int64_t i = 0; i < num_nodes; ++i) {
    const annc_hlo_node& nd = nodes[i];
    ANNC_REQUIRE(nd.rank >= 0 && nd.rank <= ANNC_HLO_MAX_RANK, "node %lld: rank out of range",
                 (long long)i);
    ANNC_REQUIRE(nd.num_operands >= 0 && nd.num_operands <= ANNC_HLO_MAX_OPERANDS,
                 "node %lld: operand count out of range", (long long)i);
    for (int k = 0; k < nd.num_operands; ++k)
      ANNC_REQUIRE(nd.operands[k] >= -1 && nd.operands[k] < num_nodes,
                   "node %lld: operand %d out of range", (long long)i, k);
  }
  std::memset(out, 0, sizeof(*out));
  Graph g{nodes, num_nodes, std::vector<std::vector<int32_t>>(num_nodes)};
  for (int64_t i = 0; i < num_nodes; ++i)
    for (int k = 0; k < nodes[i].num_operands; ++k) {
      const int32_t o = nodes[i].operands[k];
      auto& u = g.users[o < 0 ? 0 : o];
      if (o >= 0 && std::find(u.begin(), u.end(), (int32_t)i) == u.end()) u.push_back((int32_t)i);
    }
  // KDnnRewriter::execute (kdnn_rewriter.cc:44-47)
  if (nodes[instr].has_control_deps) return set_error(ANNC_OK, "");
  for (const Rewriter& rw : rewriters_for(nodes[instr].opcode)) {
    Result r;
    r.benefit = rw.benefit;
    if (rw.custom) {
      if (!rw.custom(g, instr, r)) continue;
    } else {
      if (!match_pattern(g, instr, rw.pattern, r.fused)) continue;
      r.target = rw.name;
      r.custom_call = rw.dnn_custom_call;
      r.operands = fusion_operands(g, r.fused);
      // add_extra_operands (hlo_util.h:23-33): one shape info per parameter
      r.shape_infos = r.operands;
    }
    ANNC_REQUIRE(r.fused.size() <= ANNC_HLO_MAX_FUSED && r.operands.size() <= ANNC_HLO_MAX_OPERANDS * 2 &&
                     r.shape_infos.size() <= ANNC_HLO_MAX_OPERANDS * 2,
                 "fusion too large for annc_hlo_rewrite");
    out->matched = 1;
    std::snprintf(out->target, sizeof(out->target), "%s", r.target.c_str());
    out->custom_call = r.custom_call ? 1 : 0;
    out->benefit = r.benefit;
    out->num_fused = static_cast<int32_t>(r.fused.size());
    std::copy(r.fused.begin(), r.fused.end(), out->fused);
    out->num_operands = static_cast<int32_t>(r.operands.size());
    std::copy(r.operands.begin(), r.operands.end(), out->operands);
    out->num_shape_infos = static_cast<int32_t>(r.shape_infos.size());
    std::copy(r.shape_infos.begin(), r.shape_infos.end(), out->shape_info_of);
    return set_error(ANNC_OK, "");
  }
  return set_error(ANNC_OK, "");
}
