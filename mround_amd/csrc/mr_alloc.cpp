// Exact mixed-precision bit allocation, host code.
//
// A multiple-choice knapsack: one option (bit width) per layer, minimizing
// the summed predicted loss with the summed storage cost within a budget
// (mround/planner/allocator.py:98-194). Dynamic programming over exact
// cumulative costs (no bucketing). After each layer the states are cut to the
// Pareto frontier: ascending cost with strictly falling loss. That cut is
// exact, because every remaining layer adds the same options to every state.
//
// Ties resolve as the reference's dictionary walk does. States are visited in
// ascending cost and options in the given order. A later candidate replaces
// an earlier one at the same cost only with strictly lower loss. The final
// pick is the lowest loss, then the lowest cost. Losses accumulate in double
// in the same order, so the chosen widths match the reference's exactly.
//
// Every layer's frontier is kept as (cost, loss, parent, option) records, so
// the answer is recovered by walking parents back, not by carrying a path per
// state.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <unordered_map>
#include <vector>

namespace mr {
int fail(int code, const char* fmt, ...);
void clear_error();
}  // namespace mr

namespace {

constexpr int kOk = 0;
constexpr int kEinval = -22;

struct State {
  int64_t cost;
  double loss;
  int32_t parent;  // index in the previous layer's frontier
  int32_t option;  // option index within this layer
};

// Evenly spaced ranks of the cost-sorted frontier; the cheapest state always
// survives and, from two states up, the most expensive (lowest loss) one too.
// std::nearbyint rounds half to even, as Python's round() does.
std::vector<State> thin(const std::vector<State>& f, int64_t max_states) {
  if (static_cast<int64_t>(f.size()) <= max_states) return f;
  std::vector<size_t> pick;
  if (max_states == 1) {
    pick.push_back(0);
  } else {
    const double step = static_cast<double>(f.size() - 1) / static_cast<double>(max_states - 1);
    for (int64_t i = 0; i < max_states; ++i)
      pick.push_back(static_cast<size_t>(std::nearbyint(static_cast<double>(i) * step)));
    std::sort(pick.begin(), pick.end());
    pick.erase(std::unique(pick.begin(), pick.end()), pick.end());
  }
  std::vector<State> out;
  out.reserve(pick.size());
  for (size_t i : pick) out.push_back(f[i]);
  return out;
}

}  // namespace

extern "C" {

int mr_allocate_bits(int n_layers, const int32_t* n_options, const int64_t* cost_bits,
                     const double* delta_loss, int64_t budget_bits, int64_t max_states,
                     int32_t* choice_out, double* loss_out, int64_t* cost_out) {
  mr::clear_error();
  if (n_layers <= 0) return mr::fail(kEinval, "no layers to allocate");
  if (!n_options || !cost_bits || !delta_loss || !choice_out)
    return mr::fail(kEinval, "mr_allocate_bits: null pointer");
  if (max_states < 0) return mr::fail(kEinval, "max_states must be positive or None, got %lld",
                                      static_cast<long long>(max_states));
  int64_t total_options = 0, cheapest = 0;
  for (int i = 0; i < n_layers; ++i) {
    if (n_options[i] <= 0) return mr::fail(kEinval, "layer %d has no candidate bit widths", i);
    int64_t lo = INT64_MAX;
    for (int o = 0; o < n_options[i]; ++o) {
      const int64_t c = cost_bits[total_options + o];
      const double l = delta_loss[total_options + o];
      if (c < 0) return mr::fail(kEinval, "cost_bits must be non-negative");
      if (!std::isfinite(l) || l < 0.0)
        return mr::fail(kEinval, "delta_loss must be finite and non-negative");
      lo = std::min(lo, c);
    }
    cheapest += lo;
    total_options += n_options[i];
  }
  if (cheapest > budget_bits)
    return mr::fail(kEinval,
                    "budget of %lld bits is infeasible: the cheapest possible allocation costs "
                    "%lld bits",
                    static_cast<long long>(budget_bits), static_cast<long long>(cheapest));

  std::vector<std::vector<State>> layers(n_layers);
  std::vector<State> frontier{{0, 0.0, -1, -1}};
  int64_t off = 0;
  for (int i = 0; i < n_layers; ++i) {
    std::vector<State> cand;
    std::unordered_map<int64_t, size_t> at;
    cand.reserve(frontier.size() * static_cast<size_t>(n_options[i]));
    at.reserve(frontier.size() * static_cast<size_t>(n_options[i]));
    for (size_t s = 0; s < frontier.size(); ++s) {
      for (int o = 0; o < n_options[i]; ++o) {
        const int64_t c = frontier[s].cost + cost_bits[off + o];
        if (c > budget_bits) continue;
        const double l = frontier[s].loss + delta_loss[off + o];
        auto it = at.find(c);
        if (it == at.end()) {
          at.emplace(c, cand.size());
          cand.push_back({c, l, static_cast<int32_t>(s), o});
        } else if (l < cand[it->second].loss) {
          cand[it->second] = {c, l, static_cast<int32_t>(s), o};
        }
      }
    }
    if (cand.empty())
      return mr::fail(kEinval, "no feasible allocation remains after layer %d", i);
    std::sort(cand.begin(), cand.end(),
              [](const State& a, const State& b) { return a.cost < b.cost; });
    std::vector<State> kept;
    double best = INFINITY;
    for (const State& st : cand) {
      if (st.loss < best) {
        kept.push_back(st);
        best = st.loss;
      }
    }
    if (max_states > 0) kept = thin(kept, max_states);
    layers[i] = kept;
    frontier = std::move(kept);
    off += n_options[i];
  }

  size_t best = 0;
  for (size_t s = 1; s < frontier.size(); ++s) {
    const State& a = frontier[s];
    const State& b = frontier[best];
    if (a.loss < b.loss || (a.loss == b.loss && a.cost < b.cost)) best = s;
  }
  if (loss_out) *loss_out = frontier[best].loss;
  if (cost_out) *cost_out = frontier[best].cost;
  int32_t idx = static_cast<int32_t>(best);
  for (int i = n_layers - 1; i >= 0; --i) {
    const State& st = layers[i][static_cast<size_t>(idx)];
    choice_out[i] = st.option;
    idx = st.parent;
  }
  return kOk;
}

}  // extern "C"
