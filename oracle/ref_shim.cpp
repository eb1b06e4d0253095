// ref_shim.cpp -- C entry points over the reference's own CPU path, compiled
// from the reference sources where they lie (see oracle/Makefile).  TEST
// INFRASTRUCTURE ONLY: used to write tests/golden fixtures and, optionally, as
// bench.py's CPU baseline.  Never linked into the product library.
//
// Calls (reference file:line):
//   lightning_core::attentionForwardWithPolicy   src/attention.cpp:137-201
//   lightning_core::attentionTrainStep           src/attention.cpp:203-214
//   lightning_core::ops::matMul<float>           include/lightning_core/core/ops.hpp:195-205
//   lightning_core::ops::conv2dNchw<float>       include/lightning_core/core/ops.hpp:855-1213
//   lightning_core::graph::GraphIR                include/lightning_core/core/graph.hpp:618-1790
// all with Device::kCPU (the graph planner sees the host build's devices).
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "lightning_core/core/attention.hpp"
#include "lightning_core/core/graph.hpp"
#include "lightning_core/core/ops.hpp"

namespace lc = lightning_core;

extern "C" {

int ref_attention_forward(const float* q, const float* k, const float* v, float* out, size_t s, size_t d,
                          int causal, float out_scale, float out_bias, int out_relu) {
  lc::AttentionConfig cfg{s, d, causal != 0};
  lc::AttentionIoPolicy policy;
  policy.output_scale = out_scale;
  policy.output_bias = out_bias;
  policy.output_relu = out_relu != 0;
  return static_cast<int>(lc::attentionForwardWithPolicy(q, k, v, out, cfg, lc::runtime::Device::kCPU, policy));
}

// attentionTrainStep (src/attention.cpp:203-214) on the CPU device: v is
// updated in place, *loss receives the mean squared error.
int ref_attention_train_step(const float* q, const float* k, float* v, const float* target, float* out, size_t s,
                             size_t d, int causal, float learning_rate, float* loss) {
  lc::AttentionConfig cfg{s, d, causal != 0};
  return static_cast<int>(
      lc::attentionTrainStep(q, k, v, target, out, learning_rate, cfg, lc::runtime::Device::kCPU, loss));
}

int ref_matmul(const float* a, const float* b, float* out, size_t m, size_t k, size_t n) {
  return static_cast<int>(lc::ops::matMul<float>(a, b, out, m, k, n, lc::runtime::Device::kCPU));
}

int ref_conv2d_nchw(const float* x, const float* w, const float* bias, float* out, size_t batch, size_t in_c,
                    size_t in_h, size_t in_w, size_t out_c, size_t kh, size_t kw, size_t sh, size_t sw,
                    size_t ph, size_t pw, int relu) {
  return static_cast<int>(lc::ops::conv2dNchw<float>(x, w, bias, out, batch, in_c, in_h, in_w, out_c, kh, kw, sh,
                                                     sw, ph, pw, lc::runtime::Device::kCPU, relu != 0));
}

// The reference's conv->attention chain (bind_integrated.cpp:614-730) lives in
// a pybind translation unit; this composes the same steps from the reference's
// conv2dNchw and attentionForward with the flat-slice / repeat packing.
int ref_conv_attention(const float* x, const float* w, const float* bias, float* out, size_t batch, size_t in_c,
                       size_t in_h, size_t in_w, size_t out_c, size_t kh, size_t kw, size_t seq_len,
                       size_t head_dim, size_t sh, size_t sw, size_t ph, size_t pw) {
  const size_t out_h = (in_h + 2 * ph - kh) / sh + 1;
  const size_t out_w = (in_w + 2 * pw - kw) / sw + 1;
  const size_t conv_size = batch * out_c * out_h * out_w;
  std::vector<float> conv(conv_size);
  int st = ref_conv2d_nchw(x, w, bias, conv.data(), batch, in_c, in_h, in_w, out_c, kh, kw, sh, sw, ph, pw, 1);
  if (st != 0) {
    return st;
  }
  const size_t need = seq_len * head_dim;
  const size_t total = 3 * need;
  std::vector<float> packed(total);
  size_t copied = conv_size < total ? conv_size : total;
  std::memcpy(packed.data(), conv.data(), copied * sizeof(float));
  while (copied < total) {
    const size_t chunk = copied < total - copied ? copied : total - copied;
    std::memcpy(packed.data() + copied, packed.data(), chunk * sizeof(float));
    copied += chunk;
  }
  lc::AttentionConfig cfg{seq_len, head_dim, false};
  return static_cast<int>(lc::attentionForward(packed.data(), packed.data() + need, packed.data() + 2 * need, out,
                                               cfg, lc::runtime::Device::kCPU));
}

// ---- graph IR ---------------------------------------------------------------
// The reference GraphIR behind a small C surface: reports come back as JSON in
// the layout the reference's Python binding builds (bind_graph.cpp:80-226), so
// tests can compare them with the HIP backend's reports field by field.
struct RefGraph {
  lc::graph::GraphIR g;
  std::string report;
};

}  // extern "C"

namespace {

namespace g = lc::graph;

std::string js(const std::string& s) {
  std::string o = "\"";
  for (char c : s) {
    if (c == '"' || c == '\\') {
      o += '\\';
    }
    o += c;
  }
  return o + "\"";
}
std::string jb(bool b) { return b ? "true" : "false"; }
std::string jd(double v) {
  // The reference flags include -ffast-math, under which std::isfinite folds
  // to true: test the exponent bits instead.
  std::uint64_t bits;
  std::memcpy(&bits, &v, sizeof bits);
  if (((bits >> 52) & 0x7ff) == 0x7ff) {
    return "null";
  }
  char buf[64];
  std::snprintf(buf, sizeof buf, "%.17g", v);
  return buf;
}
template <typename T>
std::string jl(const std::vector<T>& v) {
  std::string o = "[";
  for (size_t i = 0; i < v.size(); ++i) {
    o += (i ? "," : "") + std::to_string(v[i]);
  }
  return o + "]";
}
const char* dev(lc::runtime::Device d) {
  switch (d) {
    case lc::runtime::Device::kCUDA: return "cuda";
    case lc::runtime::Device::kMetal: return "metal";
    default: return "cpu";
  }
}
bool parseDevice(const std::string& s, lc::runtime::Device* d) {
  if (s == "cpu") *d = lc::runtime::Device::kCPU;
  else if (s == "cuda") *d = lc::runtime::Device::kCUDA;
  else if (s == "metal") *d = lc::runtime::Device::kMetal;
  else return false;
  return true;
}

std::string stepsJson(const std::vector<g::GraphPlanStep>& steps) {
  std::string o = "[";
  for (size_t i = 0; i < steps.size(); ++i) {
    const auto& s = steps[i];
    o += (i ? "," : "");
    o += "{\"node_id\":" + std::to_string(s.node_id) + ",\"op\":" + js(g::opKindName(s.op)) +
         ",\"assigned_device\":" + js(dev(s.assigned_device)) + ",\"fallback\":" + jb(s.fallback) +
         ",\"fallback_reason_code\":" + js(s.fallback_reason_code) + ",\"fallback_reason\":" +
         js(s.fallback_reason) + "}";
  }
  return o + "]";
}
std::string groupsJson(const std::vector<g::GraphExecutionGroup>& groups) {
  std::string o = "[";
  for (size_t i = 0; i < groups.size(); ++i) {
    const auto& gr = groups[i];
    o += (i ? "," : "");
    o += "{\"group_id\":" + std::to_string(gr.group_id) + ",\"assigned_device\":" + js(dev(gr.assigned_device)) +
         ",\"fallback\":" + jb(gr.fallback) + ",\"fallback_reason_code\":" + js(gr.fallback_reason_code) +
         ",\"fallback_reason\":" + js(gr.fallback_reason) + ",\"sync_boundary_before\":" +
         jb(gr.sync_boundary_before) + ",\"sync_boundary_after\":" + jb(gr.sync_boundary_after) +
         ",\"node_ids\":" + jl(gr.node_ids) + "}";
  }
  return o + "]";
}
std::string summaryJson(const g::GraphPlanSummary& s) {
  return "{\"total_nodes\":" + std::to_string(s.total_nodes) + ",\"total_groups\":" + std::to_string(s.total_groups) +
         ",\"planned_dispatch_groups\":" + std::to_string(s.planned_dispatch_groups) +
         ",\"total_fallback_nodes\":" + std::to_string(s.total_fallback_nodes) +
         ",\"total_fallback_groups\":" + std::to_string(s.total_fallback_groups) +
         ",\"sync_boundary_before_groups\":" + std::to_string(s.sync_boundary_before_groups) +
         ",\"sync_boundary_after_groups\":" + std::to_string(s.sync_boundary_after_groups) +
         ",\"device_switches\":" + std::to_string(s.device_switches) + ",\"cpu_nodes\":" +
         std::to_string(s.cpu_nodes) + ",\"cuda_nodes\":" + std::to_string(s.cuda_nodes) + ",\"metal_nodes\":" +
         std::to_string(s.metal_nodes) + ",\"cpu_groups\":" + std::to_string(s.cpu_groups) + ",\"cuda_groups\":" +
         std::to_string(s.cuda_groups) + ",\"metal_groups\":" + std::to_string(s.metal_groups) +
         ",\"plan_cache_enabled\":" + jb(s.plan_cache_enabled) + ",\"plan_cache_hit\":" + jb(s.plan_cache_hit) +
         ",\"plan_cache_hits_total\":" + std::to_string(s.plan_cache_hits_total) +
         ",\"plan_cache_misses_total\":" + std::to_string(s.plan_cache_misses_total) +
         ",\"plan_cache_hit_rate_pct\":" + jd(s.plan_cache_hit_rate_pct) + ",\"planner_score_model\":" +
         js(s.planner_score_model) + ",\"cost_profile_signature\":" + js(s.cost_profile_signature) +
         ",\"estimated_total_cost_ns\":" + jd(s.estimated_total_cost_ns) + ",\"estimated_compute_cost_ns\":" +
         jd(s.estimated_compute_cost_ns) + ",\"estimated_launch_cost_ns\":" + jd(s.estimated_launch_cost_ns) +
         ",\"estimated_transfer_cost_ns\":" + jd(s.estimated_transfer_cost_ns) + ",\"estimated_sync_cost_ns\":" +
         jd(s.estimated_sync_cost_ns) + ",\"estimated_boundary_cost_ns\":" + jd(s.estimated_boundary_cost_ns) + "}";
}

// Options as "key=value;key=value" with the Python binding's keyword names.
bool parseOptions(const char* text, g::GraphPlannerOptions* o) {
  std::string s = text != nullptr ? text : "";
  size_t pos = 0;
  while (pos < s.size()) {
    size_t end = s.find(';', pos);
    if (end == std::string::npos) end = s.size();
    const std::string kv = s.substr(pos, end - pos);
    pos = end + 1;
    const size_t eq = kv.find('=');
    if (eq == std::string::npos) continue;
    const std::string k = kv.substr(0, eq), v = kv.substr(eq + 1);
    const bool b = v == "1" || v == "true";
    if (k == "preferred_device") { if (!parseDevice(v, &o->preferred_device)) return false; }
    else if (k == "sync_mode") o->sync_policy.mode = v == "always" ? lc::runtime::SyncMode::kAlways
                                                    : v == "never" ? lc::runtime::SyncMode::kNever
                                                                   : lc::runtime::SyncMode::kAuto;
    else if (k == "trace_sync_boundary") o->sync_policy.trace_sync_boundary = b;
    else if (k == "group_by_backend_capability") o->group_by_backend_capability = b;
    else if (k == "separate_fallback_segments") o->separate_fallback_segments = b;
    else if (k == "insert_sync_on_device_change") o->insert_sync_on_device_change = b;
    else if (k == "enable_fusion_v1") o->enable_fusion_v1 = b;
    else if (k == "enable_fusion_pass_conv") o->enable_fusion_pass_conv = b;
    else if (k == "enable_fusion_pass_matmul") o->enable_fusion_pass_matmul = b;
    else if (k == "enable_fusion_pass_attention") o->enable_fusion_pass_attention = b;
    else if (k == "enable_fusion_pass_attention_qkv") o->enable_fusion_pass_attention_qkv = b;
    else if (k == "fusion_pass_order") o->fusion_pass_order = v;
    else if (k == "enable_fusion_cost_model_v1") o->enable_fusion_cost_model_v1 = b;
    else if (k == "enable_fusion_cost_model_v2") o->enable_fusion_cost_model_v2 = b;
    else if (k == "enable_plan_cache") o->enable_plan_cache = b;
    else if (k == "fusion_cost_min_speedup") o->fusion_cost_min_speedup = std::stod(v);
    else if (k == "cost_profile_signature") o->cost_profile_signature = v;
    else if (k == "cost_launch_overhead_ns") o->cost_launch_overhead_ns = std::stod(v);
    else if (k == "cost_transfer_overhead_ns") o->cost_transfer_overhead_ns = std::stod(v);
    else if (k == "cost_sync_boundary_ns") o->cost_sync_boundary_ns = std::stod(v);
    else if (k == "cost_elementwise_per_element_ns") o->cost_elementwise_per_element_ns = std::stod(v);
    else if (k == "cost_matmul_per_mac_ns") o->cost_matmul_per_mac_ns = std::stod(v);
    else if (k == "cost_conv_per_mac_ns") o->cost_conv_per_mac_ns = std::stod(v);
    else if (k == "planner_cost_weight_compute") o->planner_cost_weight_compute = std::stod(v);
    else if (k == "planner_cost_weight_boundary") o->planner_cost_weight_boundary = std::stod(v);
    else if (k == "planner_cost_weight_preference") o->planner_cost_weight_preference = std::stod(v);
    else return false;
  }
  return true;
}

}  // namespace

extern "C" {

void* ref_graph_create() { return new RefGraph(); }
void ref_graph_destroy(void* p) { delete static_cast<RefGraph*>(p); }

int ref_graph_add_tensor(void* p, const int64_t* shape, size_t rank, int dtype, int layout, const char* name,
                         int constant, size_t* id) {
  g::TensorSpec spec;
  spec.shape.assign(shape, shape + rank);
  spec.dtype = dtype == 1 ? g::DType::kFloat64 : g::DType::kFloat32;
  spec.layout = layout == 1 ? lc::Layout::kStrided : lc::Layout::kContiguous;
  return static_cast<int>(static_cast<RefGraph*>(p)->g.addTensorSpec(spec, id, name ? name : "", constant != 0));
}

int ref_graph_add_node(void* p, const char* op, const size_t* in, size_t nin, const size_t* out, size_t nout,
                       const size_t* deps, size_t ndeps, const char* name, const char* const* keys,
                       const int64_t* vals, size_t nattrs) {
  static const std::pair<const char*, g::OpKind> kinds[] = {
      {"matmul", g::OpKind::kMatMul}, {"vector_add", g::OpKind::kVectorAdd}, {"matrix_sub", g::OpKind::kMatrixSub},
      {"matrix_div", g::OpKind::kMatrixDiv}, {"attention_forward", g::OpKind::kAttentionForward},
      {"conv2d_nchw3x3", g::OpKind::kConv2dNchw3x3}, {"conv2d_nchw3x3s1p1", g::OpKind::kConv2dNchw3x3s1p1},
      {"qkv_pack_repeat", g::OpKind::kQkvPackRepeat}, {"relu", g::OpKind::kRelu}};
  for (const auto& k : kinds) {
    if (std::strcmp(k.first, op) == 0) {
      std::unordered_map<std::string, std::int64_t> attrs;
      for (size_t i = 0; i < nattrs; ++i) {
        attrs[keys[i]] = vals[i];
      }
      return static_cast<int>(static_cast<RefGraph*>(p)->g.addNode(
          k.second, std::vector<size_t>(in, in + nin), std::vector<size_t>(out, out + nout),
          std::vector<size_t>(deps, deps + ndeps), name ? name : "", attrs));
    }
  }
  return -1;
}

// what: validate | plan | plan_groups | plan_summary | fusion_report |
// execute_f32 | cache_stats | clear_cache.  Returns the call's status; the
// report is kept for ref_graph_report.
int ref_graph_call(void* p, const char* what, const char* opts, const size_t* feed_ids, const float* const* feeds,
                   const size_t* feed_sizes, size_t nfeeds) {
  RefGraph* r = static_cast<RefGraph*>(p);
  const std::string w = what;
  g::GraphPlannerOptions o;
  if (!parseOptions(opts, &o)) {
    return -1;
  }
  lc::runtime::Status st = lc::runtime::Status::kSuccess;
  if (w == "validate") {
    g::ValidationReport rep;
    st = r->g.validateWithReport(&rep);
    std::string s = "{\"ok\":" + jb(st == lc::runtime::Status::kSuccess) + ",\"status\":" +
                    js(lc::runtime::getErrorString(st)) + ",\"issues\":[";
    for (size_t i = 0; i < rep.issues.size(); ++i) {
      const auto& is = rep.issues[i];
      s += (i ? "," : "");
      s += "{\"pass\":" + js(g::validationPassName(is.pass)) + ",\"status\":" + js(lc::runtime::getErrorString(is.status)) +
           ",\"node_id\":" + std::to_string(is.node_id) + ",\"tensor_id\":" + std::to_string(is.tensor_id) +
           ",\"reason_code\":" + js(g::reasonCodeName(is.reason)) + ",\"message\":" + js(is.message) + "}";
    }
    r->report = s + "]}";
  } else if (w == "plan") {
    std::vector<g::GraphPlanStep> steps;
    st = r->g.planForDevice(o.preferred_device, &steps);
    r->report = stepsJson(steps);
  } else if (w == "plan_groups") {
    std::vector<g::GraphExecutionGroup> groups;
    std::vector<g::GraphPlanStep> steps;
    g::GraphPlanSummary sum{};
    st = r->g.planExecutionGroups(o, &groups, &steps);
    if (st == lc::runtime::Status::kSuccess) st = r->g.planSummary(o, &sum, nullptr, nullptr);
    r->report = "{\"groups\":" + groupsJson(groups) + ",\"steps\":" + stepsJson(steps) + ",\"summary\":" +
                summaryJson(sum) + "}";
  } else if (w == "plan_summary") {
    std::vector<g::GraphExecutionGroup> groups;
    std::vector<g::GraphPlanStep> steps;
    g::GraphPlanSummary sum{};
    st = r->g.planSummary(o, &sum, &groups, &steps);
    r->report = "{\"summary\":" + summaryJson(sum) + ",\"groups\":" + groupsJson(groups) + ",\"steps\":" +
                stepsJson(steps) + "}";
  } else if (w == "fusion_report") {
    std::vector<g::GraphFusionDecision> ds;
    st = r->g.fusionReport(o, &ds);
    std::string s = "[";
    for (size_t i = 0; i < ds.size(); ++i) {
      const auto& d = ds[i];
      s += (i ? "," : "");
      s += "{\"pattern\":" + js(g::fusionPatternName(d.pattern)) + ",\"pass_id\":" + js(d.pass_id) +
           ",\"pass_order\":" + std::to_string(d.pass_order) + ",\"start_node_id\":" + std::to_string(d.start_node_id) +
           ",\"end_node_id\":" + std::to_string(d.end_node_id) + ",\"assigned_device\":" + js(dev(d.assigned_device)) +
           ",\"fused\":" + jb(d.fused) + ",\"cost_model_applied\":" + jb(d.cost_model_applied) +
           ",\"estimated_unfused_cost_ns\":" + jd(d.estimated_unfused_cost_ns) + ",\"estimated_fused_cost_ns\":" +
           jd(d.estimated_fused_cost_ns) + ",\"estimated_speedup\":" + jd(d.estimated_speedup) +
           ",\"cost_profile_signature\":" + js(d.cost_profile_signature) + ",\"reason\":" + js(d.reason) + "}";
    }
    r->report = s + "]";
  } else if (w == "execute_f32") {
    std::unordered_map<size_t, std::vector<float>> in, vals;
    for (size_t i = 0; i < nfeeds; ++i) {
      in[feed_ids[i]] = std::vector<float>(feeds[i], feeds[i] + feed_sizes[i]);
    }
    std::vector<g::GraphExecutionGroup> groups;
    std::vector<g::GraphPlanStep> steps;
    g::GraphPlanSummary sum{};
    st = r->g.executeF32(o, in, &vals, &groups, &steps);
    if (st == lc::runtime::Status::kSuccess) st = r->g.planSummary(o, &sum, nullptr, nullptr);
    std::string s = "{\"values\":{";
    size_t k = 0;
    for (const auto& kv : vals) {
      s += (k++ ? ",\"" : "\"") + std::to_string(kv.first) + "\":[";
      for (size_t i = 0; i < kv.second.size(); ++i) {
        char buf[32];
        std::snprintf(buf, sizeof buf, "%s%.9g", i ? "," : "", static_cast<double>(kv.second[i]));
        s += buf;
      }
      s += "]";
    }
    r->report = s + "},\"groups\":" + groupsJson(groups) + ",\"steps\":" + stepsJson(steps) + ",\"summary\":" +
                summaryJson(sum) + "}";
  } else if (w == "registry") {
    std::string s = "[";
    const auto schemas = g::globalOperatorRegistry().schemas();
    for (size_t i = 0; i < schemas.size(); ++i) {
      const auto& sc = schemas[i];
      s += (i ? "," : "");
      s += "{\"op\":" + js(g::opKindName(sc.kind)) + ",\"name\":" + js(sc.name) + ",\"min_inputs\":" +
           std::to_string(sc.min_inputs) + ",\"max_inputs\":" + std::to_string(sc.max_inputs) +
           ",\"min_outputs\":" + std::to_string(sc.min_outputs) + ",\"max_outputs\":" +
           std::to_string(sc.max_outputs) + ",\"supports_cpu\":" + jb(sc.supports_cpu) + ",\"supports_cuda\":" +
           jb(sc.supports_cuda) + ",\"supports_metal\":" + jb(sc.supports_metal) + ",\"input_ranks\":" +
           jl(sc.input_ranks) + ",\"output_ranks\":" + jl(sc.output_ranks) + ",\"allow_float32\":" +
           jb(sc.allow_float32) + ",\"allow_float64\":" + jb(sc.allow_float64) +
           ",\"require_contiguous_layout\":" + jb(sc.require_contiguous_layout) + ",\"allowed_attributes\":[";
      size_t k = 0;
      for (const auto& a : sc.allowed_attributes) {
        s += (k++ ? "," : "") + js(a);
      }
      s += "]}";
    }
    r->report = s + "]";
  } else if (w == "cache_stats") {
    const auto cs = r->g.planCacheStats();
    r->report = "{\"hits\":" + std::to_string(cs.hits) + ",\"misses\":" + std::to_string(cs.misses) +
                ",\"hit_rate_pct\":" + jd(cs.hit_rate_pct) + "}";
  } else if (w == "clear_cache") {
    r->g.clearPlanCache();
    r->report = "{}";
  } else {
    return -1;
  }
  return static_cast<int>(st);
}

size_t ref_graph_report(void* p, char* buf, size_t cap) {
  const std::string& s = static_cast<RefGraph*>(p)->report;
  if (buf != nullptr && cap > s.size()) {
    std::memcpy(buf, s.c_str(), s.size() + 1);
  }
  return s.size() + 1;
}

}  // extern "C"
