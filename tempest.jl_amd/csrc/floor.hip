// Op class (a), generated: the floor's kernels for any pointwise or reduction
// group, written from the group's terms, compiled at run time for gfx950 and
// kept in a content-keyed code-object cache.
//
// The reference generates a Julia function per group (scalar_kernel,
// src/Compiler/codegen/scalar.jl:186-250; split_kernels, :284-348) and CUDA
// runs it one thread per item, or dealt over Split(parts, lanes, side)
// (floor_launch / floor_split / merge_lanes, ext/CUDAExt.jl:926-1017).  Here
// the group arrives through the C ABI as plain arrays (th_floor_desc) and the
// kernel is HIP source written for CDNA4:
//   * rows: an item's positions are adjacent in memory, so one workgroup of
//     64-256 lanes sweeps an item, four positions a lane at a time with
//     16-byte loads, merges its lanes by wave shuffles and LDS, and, when an
//     item's positions fit, keeps every load in registers across the phases
//     (each element read once from HBM);
//   * columns: neighbouring items are adjacent in memory, so a wave holds 64
//     items side by side, each thread sweeping its item's positions (or a
//     share of them, merged through LDS);
//   * few items: the positions split into parts (workgroups), each part's
//     state goes to a workspace, and the next launch merges the parts.
// Phases run in one kernel when an item fits one workgroup; split folds take
// a launch per phase and one after them, as the reference's split kernels do.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <dirent.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cinttypes>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <deque>
#include <fstream>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <unordered_map>
#include <vector>

#include "th_core.h"

namespace th {
namespace floorgen {

constexpr int kRank = TH_FLOOR_RANK;
constexpr int kMaxArgs = 64;        // pointers in a kernel's argument struct (512 bytes)
constexpr int kCUs = 256;           // MI355X
constexpr int kResidentFloats = 128;  // registers a thread may spend keeping loads
constexpr int kMaxIters = 32;

int arity(int fn) {
  switch (fn) {
    case TH_FN_ADD: case TH_FN_SUB: case TH_FN_MUL: case TH_FN_DIV: case TH_FN_POW:
    case TH_FN_MAX: case TH_FN_MIN: case TH_FN_LT: case TH_FN_LE: case TH_FN_GT:
    case TH_FN_GE: case TH_FN_EQ: case TH_FN_NE:
      return 2;
    case TH_FN_IFELSE: case TH_FN_CLAMP: case TH_FN_FMA: case TH_FN_DROPOUT:
      return 3;
    default:
      return fn >= 0 && fn < TH_FN_COUNT ? 1 : -1;
  }
}

const char* fn_name(int fn) {
  static const char* names[TH_FN_COUNT] = {
      "", "", "", "", "", "th_abs", "th_abs2", "th_sqrt", "th_exp", "th_log", "th_tanh", "th_sin",
      "th_cos", "th_log1p", "th_expm1", "th_pow", "th_max", "th_min", "th_lt", "th_le", "th_gt",
      "th_ge", "th_eq", "th_ne", "th_ifelse", "th_round", "th_floor", "th_ceil", "th_sign",
      "th_clamp", "th_fma", "th_inv", "th_rbf", "th_dropout"};
  return names[fn];
}

// Components of a fold's state.
int state_size(int kind) {
  return kind == TH_FOLD_EXP || kind == TH_FOLD_LINEAR || kind == TH_FOLD_ARGMAX || kind == TH_FOLD_ARGMIN ? 2
         : kind == TH_FOLD_SQUARE ? 3 : 1;
}

bool observe_ok(int kind, int obs) {
  switch (kind) {
    case TH_FOLD_EXP: return obs == TH_OBSERVE_STATISTIC || obs == TH_OBSERVE_SUM || obs == TH_OBSERVE_LOGSUMEXP;
    case TH_FOLD_SQUARE: return obs == TH_OBSERVE_STATISTIC || obs == TH_OBSERVE_SUM;
    case TH_FOLD_LINEAR:
    case TH_FOLD_ARGMAX:
    case TH_FOLD_ARGMIN: return obs == TH_OBSERVE_VALUE || obs == TH_OBSERVE_STATISTIC;
    default: return obs == TH_OBSERVE_VALUE;
  }
}

std::string flt(float x) {
  if (std::isnan(x)) return "__builtin_nanf(\"\")";
  if (std::isinf(x)) return x > 0 ? "__builtin_inff()" : "(-__builtin_inff())";
  char b[64];
  std::snprintf(b, sizeof b, "(%af)", (double)x);
  return b;
}

// How a group maps onto the device.
struct Plan {
  const th_floor_desc* d = nullptr;
  bool reduction = false;        // a reduction or a scan group: items sweep their folded axes
  bool recurrence = false;       // a recurrence group: a thread per item steps along `step`
  int step = -1;                 // the recurrence's step axis
  bool scan = false;             // a scan group: one thread per item, in order
  bool reverse = false;
  bool ordered = false;           // one thread takes the items in order (TH_FLOOR_ORDERED)
  std::vector<int> order;        // a scan group's folds in (phase, index) order
  int rank = 1;
  int64_t E[kRank] = {1, 1, 1, 1};
  std::vector<int> kept, swept;  // axes, fastest first
  int64_t items = 1, count = 1;  // items; positions an item folds (pointwise: 1)
  bool rows = true;              // positions adjacent (rows) or items adjacent (columns)
  int S = 1, L = 1, P = 1, W = 1;
  int vax = -1;                  // the axis W positions run along
  int64_t qn = 0;                // W-position chunks an item folds (pointwise: chunks in all)
  bool resident = false;
  int iters = 0;
  std::vector<int> phases;
  std::vector<char> dep;         // term reads the swept positions
  std::vector<char> vec_ok;      // per value: 16-byte (f32) / 8-byte (bf16) accesses allowed
  std::vector<char> written, read;
  bool gathers = false;          // some address is data-dependent: width 1, nothing kept in registers
};

bool is_int(int dtype) { return dtype == TH_I32 || dtype == TH_I64; }
int esize(int dtype) { return dtype == TH_BF16 ? 2 : dtype == TH_I64 ? 8 : 4; }

// A div or mod atom is well formed: a known kind and a positive divisor.
bool parts_ok(const th_affine& a) {
  for (const th_part& q : a.part) {
    if (q.kind == TH_PART_NONE) continue;
    if ((q.kind != TH_PART_DIV && q.kind != TH_PART_MOD) || q.divisor <= 0) return false;
  }
  return true;
}

int64_t fld(int64_t x, int64_t d) { return x >= 0 ? x / d : -((-x + d - 1) / d); }

// The least and greatest of constant + sum coeff[k] i_k over the domain.
void span(int64_t constant, const int64_t* coeff, const int64_t* ext, int rank, int64_t& lo, int64_t& hi) {
  lo = hi = constant;
  for (int k = 0; k < rank; ++k) {
    const int64_t c = coeff[k] * (ext[k] - 1);
    if (c < 0) lo += c; else hi += c;
  }
}

// The range of a part's atom (before its coefficient) over the domain.
void part_span(const th_part& q, const int64_t* ext, int rank, int64_t& lo, int64_t& hi) {
  span(q.constant, q.inner, ext, rank, lo, hi);
  if (q.kind == TH_PART_DIV) {
    lo = fld(lo, q.divisor), hi = fld(hi, q.divisor);
  } else if (fld(lo, q.divisor) == fld(hi, q.divisor)) {  // no wrap: an interval of remainders
    lo -= fld(lo, q.divisor) * q.divisor, hi -= fld(hi, q.divisor) * q.divisor;
  } else {
    lo = 0, hi = q.divisor - 1;
  }
}

bool in_box(const th_affine& a, const int64_t* ext, int rank, int64_t length) {
  if (a.gather >= 0) return true;  // data-dependent: clamped on the device
  for (int k = 0; k < rank; ++k)
    if (ext[k] <= 0) return true;  // an empty domain reads nothing
  int64_t lo, hi;
  span(a.constant, a.coeff, ext, rank, lo, hi);
  for (const th_part& q : a.part) {
    if (q.kind == TH_PART_NONE || q.coeff == 0) continue;
    int64_t plo, phi;
    part_span(q, ext, rank, plo, phi);
    if (q.coeff > 0) lo += q.coeff * plo, hi += q.coeff * phi;
    else lo += q.coeff * phi, hi += q.coeff * plo;
  }
  return lo >= 0 && hi < length;
}

bool has_parts(const th_affine& a) { return a.part[0].kind != TH_PART_NONE || a.part[1].kind != TH_PART_NONE; }

std::vector<char> reach(const th_floor_desc* d, const std::vector<int>& roots);

// The step axis of a recurrence group, from its flags.
int step_axis(const th_floor_desc* d) { return (d->flags >> 8) & 7; }

int validate(const th_floor_desc* d) {
  TH_REQUIRE(d != nullptr, "th_build_floor: null description");
  TH_REQUIRE(d->kind == TH_GROUP_POINTWISE || d->kind == TH_GROUP_REDUCTION || d->kind == TH_GROUP_SCAN ||
                 d->kind == TH_GROUP_RECURRENCE,
             "th_build_floor: unknown group kind");
  const bool rec = d->kind == TH_GROUP_RECURRENCE;
  TH_REQUIRE(d->flags == 0 || (d->kind == TH_GROUP_SCAN && d->flags == TH_FLOOR_REVERSE) ||
                 (rec && (d->flags & ~(TH_FLOOR_REVERSE | TH_FLOOR_STEP(7))) == 0) ||
                 (d->kind == TH_GROUP_POINTWISE && d->flags == TH_FLOOR_ORDERED),
             "th_build_floor: only a scan or a recurrence group runs in reverse, only a pointwise one in order");
  TH_REQUIRE(d->rank >= 1 && d->rank <= kRank, "th_build_floor: rank must be 1..4");
  for (int k = 0; k < d->rank; ++k) TH_REQUIRE(d->extents[k] >= 0, "th_build_floor: negative extent");
  const uint32_t all = (1u << d->rank) - 1;
  TH_REQUIRE(d->n_folds == 0 || d->folds, "th_build_floor: null folds");
  int stepped = 0;  // folds run in phases (not recomputed where read)
  for (int f = 0; f < d->n_folds; ++f) stepped += d->folds[f].phase >= 1;
  if (d->kind == TH_GROUP_REDUCTION || d->kind == TH_GROUP_SCAN) {
    TH_REQUIRE(d->reduced != 0 && (d->reduced & ~all) == 0, "th_build_floor: a reduction folds some of its axes");
    TH_REQUIRE(stepped >= 1, "th_build_floor: a reduction group has folds");
  } else if (rec) {
    TH_REQUIRE(step_axis(d) < d->rank && (d->reduced >> step_axis(d) & 1) && (d->reduced & ~all) == 0,
               "th_build_floor: a recurrence steps along one of its reduced axes");
    TH_REQUIRE(stepped == 0, "th_build_floor: a recurrence group's folds are recomputed where read");
  } else {
    TH_REQUIRE(d->reduced == 0 && stepped == 0, "th_build_floor: a pointwise group folds nothing");
  }
  TH_REQUIRE(d->n_values >= 1 && d->values, "th_build_floor: no values");
  TH_REQUIRE(d->n_terms >= 1 && d->terms, "th_build_floor: no terms");
  TH_REQUIRE(d->n_outputs >= 1 && d->outputs, "th_build_floor: no outputs");
  const int nws = d->kind == TH_GROUP_REDUCTION ? d->n_folds : 0;
  TH_REQUIRE(d->n_values + nws <= kMaxArgs, "th_build_floor: more than 64 values and folds");
  for (int v = 0; v < d->n_values; ++v) {
    const th_floor_value& x = d->values[v];
    TH_REQUIRE(x.dtype == TH_F32 || x.dtype == TH_BF16 || is_int(x.dtype),
               "th_build_floor: values are fp32, bf16, or int32 / int64 indices");
    TH_REQUIRE(x.length >= 0, "th_build_floor: negative value length");
    TH_REQUIRE(x.ptr != nullptr, "th_build_floor: null value pointer");
  }
  // A gathered address adds an earlier term's value: a load of integers.
  auto gather_ok = [&](const th_affine& a, int before) {
    if (a.gather < 0) return true;
    if (a.gather >= before || a.gather >= d->n_terms) return false;
    const th_term& g = d->terms[a.gather];
    // Integers, or floats holding integers (an extreme's index), truncated.
    return g.op == TH_TERM_LOAD && g.ref >= 0 && g.ref < d->n_values;
  };
  for (int t = 0; t < d->n_terms; ++t) {
    const th_term& m = d->terms[t];
    std::string at = "th_build_floor: term " + std::to_string(t) + ": ";
    TH_REQUIRE(m.op == TH_TERM_LOAD ? gather_ok(m.index, t) : m.index.gather < 0,
               at + "a gathered address adds an earlier load");
    TH_REQUIRE(parts_ok(m.index), at + "a div or mod atom takes a positive divisor");
    switch (m.op) {
      case TH_TERM_LOAD:
        TH_REQUIRE(m.ref >= 0 && m.ref < d->n_values, at + "load of no value");
        TH_REQUIRE(in_box(m.index, d->extents, d->rank, d->values[m.ref].length),
                   at + "load outside its value over the domain");
        break;
      case TH_TERM_LIT:
      case TH_TERM_INDEX:
        break;
      case TH_TERM_STAT:
        TH_REQUIRE(d->kind != TH_GROUP_POINTWISE && !rec, at + "statistic in a pointwise or recurrence group");
        TH_REQUIRE(m.ref >= 0 && m.ref < d->n_folds, at + "statistic of no fold");
        TH_REQUIRE(d->folds[m.ref].phase >= 1, at + "a statistic reads a fold run in a phase");
        TH_REQUIRE(observe_ok(d->folds[m.ref].kind, m.observe), at + "the fold has no such observation");
        break;
      case TH_TERM_RECOMPUTE:
        TH_REQUIRE(m.ref >= 0 && m.ref < d->n_folds, at + "recomputes no fold");
        TH_REQUIRE(d->folds[m.ref].phase == 0, at + "a recomputed fold has phase 0");
        TH_REQUIRE(d->folds[m.ref].body < t && d->folds[m.ref].weight < t,
                   at + "a recomputed fold's body is an earlier term");
        TH_REQUIRE(observe_ok(d->folds[m.ref].kind, m.observe), at + "the fold has no such observation");
        break;
      case TH_TERM_APPLY: {
        int n = arity(m.fn);
        TH_REQUIRE(n > 0, at + "unknown function");
        for (int j = 0; j < n; ++j)
          TH_REQUIRE(m.args[j] >= 0 && m.args[j] < t, at + "arguments must be earlier terms");
        break;
      }
      default:
        return fail(TH_E_ARGUMENT, at + "unknown term");
    }
  }
  for (int f = 0; f < d->n_folds; ++f) {
    const th_fold& x = d->folds[f];
    std::string at = "th_build_floor: fold " + std::to_string(f) + ": ";
    TH_REQUIRE(x.kind >= TH_FOLD_SUM && x.kind <= TH_FOLD_ARGMIN, at + "unknown fold");
    const bool weighted = x.kind == TH_FOLD_EXP || x.kind == TH_FOLD_LINEAR || x.kind == TH_FOLD_ARGMAX ||
                          x.kind == TH_FOLD_ARGMIN;
    TH_REQUIRE(x.phase >= 1 || (x.phase == 0 && x.scan == TH_SCAN_NONE && x.n_inner >= 1 &&
                                 d->rank + x.n_inner <= kRank),
               at + "phases start at 1; a recomputed fold (phase 0) sweeps 1..4 - rank axes of its own");
    if (x.phase == 0)
      for (int k = 0; k < x.n_inner; ++k) TH_REQUIRE(x.inner[k] >= 0, at + "negative extent");
    TH_REQUIRE(x.body >= 0 && x.body < d->n_terms, at + "no body");
    TH_REQUIRE(x.weight == -1 || (weighted && x.weight >= 0 && x.weight < d->n_terms),
               at + "only the exponential, linear and extreme folds take a weight");
    TH_REQUIRE(x.kind != TH_FOLD_LINEAR || x.weight >= 0, at + "the linear fold's weight is its offset b");
    TH_REQUIRE((x.kind != TH_FOLD_ARGMAX && x.kind != TH_FOLD_ARGMIN) || x.weight >= 0,
               at + "an extreme's weight is its element's index");
    TH_REQUIRE(x.scan == TH_SCAN_NONE || (d->kind == TH_GROUP_SCAN && x.scan <= TH_SCAN_EXCLUSIVE),
               at + "only a scan group's folds scan");
  }
  for (int o = 0; o < d->n_outputs; ++o) {
    const th_output& x = d->outputs[o];
    std::string at = "th_build_floor: output " + std::to_string(o) + ": ";
    TH_REQUIRE(x.value >= 0 && x.value < d->n_values, at + "no value");
    TH_REQUIRE(x.term >= 0 && x.term < d->n_terms, at + "no term");
    if (rec) {
      TH_REQUIRE(x.full >= TH_STEP_EACH && x.full <= TH_STEP_CARRY, at + "a recurrence output's rule is 0..3");
      TH_REQUIRE(x.accumulate == 0, at + "a recurrence stores, it does not accumulate");
      // Over the parallel axes, the step axis, and the other reduced axes its
      // address mentions (the rest at zero).  A value carried into its state
      // is written at every step but the last, its address one step on.
      const int sa = step_axis(d);
      int64_t ext[kRank];
      th_affine a = x.index;
      for (int k = 0; k < d->rank; ++k) {
        bool mentioned = a.coeff[k] != 0;
        for (const th_part& q : a.part) mentioned |= q.kind != TH_PART_NONE && q.coeff != 0 && q.inner[k] != 0;
        ext[k] = (d->reduced >> k & 1) && k != sa && !mentioned ? std::min<int64_t>(d->extents[k], 1) : d->extents[k];
      }
      if (x.full == TH_STEP_CARRY) {
        for (const th_part& q : a.part)
          TH_REQUIRE(q.kind == TH_PART_NONE || q.coeff == 0 || q.inner[sa] == 0,
                     at + "a carried value's div or mod atoms do not move along the steps");
        ext[sa] = std::max<int64_t>(d->extents[sa] - 1, 0);
        if (d->flags & TH_FLOOR_REVERSE) a.constant += a.coeff[sa];  // written at steps E-1 .. 1
      }
      TH_REQUIRE(in_box(a, ext, d->rank, d->values[x.value].length), at + "writes outside its value");
    } else {
      TH_REQUIRE(x.full == 0 || x.full == 1, at + "full is 0 or 1");
      TH_REQUIRE(x.full == 1 || d->kind != TH_GROUP_POINTWISE, at + "a pointwise group writes every position");
      // Once outputs are written with the folded positions at zero, also when
      // the folded axes are empty.
      int64_t ext[kRank];
      for (int k = 0; k < d->rank; ++k) ext[k] = (!x.full && (d->reduced >> k & 1)) ? 1 : d->extents[k];
      TH_REQUIRE(in_box(x.index, ext, d->rank, d->values[x.value].length), at + "writes outside its value");
    }
    TH_REQUIRE(gather_ok(x.index, d->n_terms), at + "a gathered address adds a load");
    TH_REQUIRE(parts_ok(x.index), at + "a div or mod atom takes a positive divisor");
    TH_REQUIRE(!is_int(d->values[x.value].dtype), at + "integer values are only read");
    TH_REQUIRE(x.accumulate == 0 || (x.accumulate == 1 && d->values[x.value].dtype == TH_F32),
               at + "accumulating outputs are fp32");
  }
  // Terms a recomputed fold's body reaches take the fold's own axes, at
  // positions rank, rank + 1, ...; no other term or output moves along them.
  std::vector<int> extra(d->n_terms, 0);
  for (int f = 0; f < d->n_folds; ++f) {
    const th_fold& x = d->folds[f];
    if (x.phase != 0) continue;
    std::vector<int> roots{x.body};
    if (x.weight >= 0) roots.push_back(x.weight);
    const std::vector<char> r = reach(d, roots);
    int64_t ext[kRank];
    for (int k = 0; k < kRank; ++k) ext[k] = k < d->rank ? d->extents[k] : (k - d->rank < x.n_inner ? x.inner[k - d->rank] : 1);
    for (int t = 0; t < d->n_terms; ++t) {
      if (!r[t]) continue;
      const th_term& m = d->terms[t];
      TH_REQUIRE(m.op != TH_TERM_RECOMPUTE, "th_build_floor: fold " + std::to_string(f) +
                                                ": a recomputed fold's body recomputes no other fold");
      extra[t] = std::max(extra[t], x.n_inner);
      if (m.op == TH_TERM_LOAD)
        TH_REQUIRE(in_box(m.index, ext, d->rank + x.n_inner, d->values[m.ref].length),
                   "th_build_floor: term " + std::to_string(t) + ": load outside its value over fold " +
                       std::to_string(f) + "'s axes");
    }
  }
  auto beyond = [&](const th_affine& a, int allowed) {
    for (int k = d->rank + allowed; k < kRank; ++k)
      if (a.coeff[k] != 0) return true;
    for (const th_part& q : a.part)
      for (int k = d->rank; k < kRank; ++k)
        if (q.kind != TH_PART_NONE && q.inner[k] != 0) return true;
    return false;
  };
  for (int t = 0; t < d->n_terms; ++t)
    TH_REQUIRE(!beyond(d->terms[t].index, extra[t]),
               "th_build_floor: term " + std::to_string(t) + ": an address moves along an axis beyond the domain");
  for (int o = 0; o < d->n_outputs; ++o)
    TH_REQUIRE(!beyond(d->outputs[o].index, 0),
               "th_build_floor: output " + std::to_string(o) + ": an address moves along an axis beyond the domain");
  if (d->kind == TH_GROUP_REDUCTION || d->kind == TH_GROUP_SCAN) {
    // Loads evaluated outside the sweep: those whose address does not move
    // along the folded axes (hoisted, read by every item even when the folded
    // positions are empty) and those the once outputs read (with the folded
    // positions at zero).
    int64_t at0[kRank];
    for (int k = 0; k < d->rank; ++k) at0[k] = (d->reduced >> k & 1) ? 1 : d->extents[k];
    std::vector<int> roots;
    for (int o = 0; o < d->n_outputs; ++o)
      if (!d->outputs[o].full) roots.push_back(d->outputs[o].term);
    const std::vector<char> once = reach(d, roots);
    for (int t = 0; t < d->n_terms; ++t) {
      const th_term& m = d->terms[t];
      if (m.op != TH_TERM_LOAD) continue;
      bool moves = false;
      for (int k = 0; k < d->rank; ++k) {
        if (!(d->reduced >> k & 1)) continue;
        moves |= m.index.coeff[k] != 0;
        for (const th_part& q : m.index.part) moves |= q.kind != TH_PART_NONE && q.coeff != 0 && q.inner[k] != 0;
      }
      if (once[t] || !moves)
        TH_REQUIRE(in_box(m.index, at0, d->rank, d->values[m.ref].length),
                   "th_build_floor: term " + std::to_string(t) +
                       ": load outside its value where it is read with the folded positions at zero");
    }
  }
  return TH_OK;
}

// Terms reachable from `roots`.
std::vector<char> reach(const th_floor_desc* d, const std::vector<int>& roots) {
  std::vector<char> r(d->n_terms, 0);
  for (int t : roots) r[t] = 1;
  for (int t = d->n_terms - 1; t >= 0; --t) {
    if (!r[t]) continue;
    if (d->terms[t].op == TH_TERM_LOAD && d->terms[t].index.gather >= 0) r[d->terms[t].index.gather] = 1;
    if (d->terms[t].op != TH_TERM_APPLY) continue;
    for (int j = 0; j < arity(d->terms[t].fn); ++j) r[d->terms[t].args[j]] = 1;
  }
  return r;
}

// Statistics a set of terms reads: the largest phase among their folds.
int max_stat_phase(const th_floor_desc* d, const std::vector<char>& r) {
  int p = 0;
  for (int t = 0; t < d->n_terms; ++t)
    if (r[t] && d->terms[t].op == TH_TERM_STAT) p = std::max(p, d->folds[d->terms[t].ref].phase);
  return p;
}

int64_t prevpow2(int64_t x) {
  int64_t p = 1;
  while (p * 2 <= x) p *= 2;
  return p;
}

int64_t nextpow2(int64_t x) {
  int64_t p = 1;
  while (p < x) p *= 2;
  return p;
}

int plan(const th_floor_desc* d, Plan& pl) {
  if (int r = validate(d)) return r;
  pl.d = d;
  pl.reduction = d->kind == TH_GROUP_REDUCTION || d->kind == TH_GROUP_SCAN;
  pl.recurrence = d->kind == TH_GROUP_RECURRENCE;
  pl.step = pl.recurrence ? step_axis(d) : -1;
  pl.scan = d->kind == TH_GROUP_SCAN;
  pl.reverse = (d->flags & TH_FLOOR_REVERSE) != 0 && d->kind != TH_GROUP_POINTWISE;
  pl.ordered = d->kind == TH_GROUP_POINTWISE && (d->flags & TH_FLOOR_ORDERED) != 0;
  pl.rank = d->rank;
  for (int k = 0; k < d->rank; ++k) pl.E[k] = d->extents[k];
  for (int k = 0; k < d->rank; ++k) ((pl.reduction && (d->reduced >> k & 1)) ? pl.swept : pl.kept).push_back(k);
  pl.items = 1;
  for (int k : pl.kept) pl.items *= pl.E[k];
  pl.count = 1;
  for (int k : pl.swept) pl.count *= pl.E[k];
  const int nt = d->n_terms;

  for (int t = 0; t < nt; ++t) pl.gathers |= d->terms[t].op == TH_TERM_LOAD && d->terms[t].index.gather >= 0;
  for (int o = 0; o < d->n_outputs; ++o) pl.gathers |= d->outputs[o].index.gather >= 0;
  // Div and mod atoms break the run of W consecutive positions: width 1, as a gather.
  for (int t = 0; t < nt; ++t) pl.gathers |= has_parts(d->terms[t].index);
  for (int o = 0; o < d->n_outputs; ++o) pl.gathers |= has_parts(d->outputs[o].index);
  // A recomputed fold sweeps its own axes in a loop: width 1, as a gather.
  for (int t = 0; t < nt; ++t) pl.gathers |= d->terms[t].op == TH_TERM_RECOMPUTE;
  // Which terms move along the swept positions.
  pl.dep.assign(nt, 0);
  for (int t = 0; t < nt; ++t) {
    const th_term& m = d->terms[t];
    if (m.op == TH_TERM_LOAD || m.op == TH_TERM_INDEX) {
      if (!pl.reduction) {
        pl.dep[t] = 1;
      } else {
        for (int k : pl.swept) pl.dep[t] |= m.index.coeff[k] != 0;
        for (const th_part& q : m.index.part)
          if (q.kind != TH_PART_NONE && q.coeff != 0)
            for (int k : pl.swept) pl.dep[t] |= q.inner[k] != 0;
        if (m.op == TH_TERM_LOAD && m.index.gather >= 0) pl.dep[t] |= pl.dep[m.index.gather];
      }
    } else if (m.op == TH_TERM_APPLY) {
      for (int j = 0; j < arity(m.fn); ++j) pl.dep[t] |= pl.dep[m.args[j]];
    } else if (m.op == TH_TERM_STAT && d->kind == TH_GROUP_SCAN) {
      pl.dep[t] = d->folds[m.ref].scan != TH_SCAN_NONE;  // a scan's result moves along the sweep
    } else if (m.op == TH_TERM_RECOMPUTE) {
      // Its body's own axes are not the swept ones: it moves where its body does.
      const th_fold& f = d->folds[m.ref];
      std::vector<int> roots{f.body};
      if (f.weight >= 0) roots.push_back(f.weight);
      const std::vector<char> r = reach(d, roots);
      for (int k = 0; k < t; ++k) pl.dep[t] |= r[k] && pl.dep[k];
    }
  }
  pl.read.assign(d->n_values, 0);
  pl.written.assign(d->n_values, 0);
  for (int t = 0; t < nt; ++t)
    if (d->terms[t].op == TH_TERM_LOAD) pl.read[d->terms[t].ref] = 1;
  for (int o = 0; o < d->n_outputs; ++o) pl.written[d->outputs[o].value] = 1;

  if (pl.scan) {
    // Folds in (phase, index) order; a fold reads only the folds before it.
    for (int f = 0; f < d->n_folds; ++f)
      if (d->folds[f].phase >= 1) pl.order.push_back(f);
    std::stable_sort(pl.order.begin(), pl.order.end(),
                     [&](int a, int b) { return d->folds[a].phase < d->folds[b].phase; });
    std::vector<int> rank_of(d->n_folds, -1);
    for (size_t j = 0; j < pl.order.size(); ++j) rank_of[pl.order[j]] = (int)j;
    for (int f : pl.order) {
      std::vector<int> roots{d->folds[f].body};
      if (d->folds[f].weight >= 0) roots.push_back(d->folds[f].weight);
      std::vector<char> r = reach(d, roots);
      for (int t = 0; t < nt; ++t)
        if (r[t] && d->terms[t].op == TH_TERM_STAT) {
          const int g = d->terms[t].ref;
          TH_REQUIRE(rank_of[g] < rank_of[f], "th_build_floor: fold " + std::to_string(f) +
                                                  " reads a fold that takes its element after it");
          TH_REQUIRE(d->folds[g].scan != TH_SCAN_NONE, "th_build_floor: fold " + std::to_string(f) +
                                                           " reads a plain fold's result inside the sweep");
        }
    }
    for (int o = 0; o < d->n_outputs; ++o) {
      std::vector<char> r = reach(d, {d->outputs[o].term});
      for (int t = 0; t < nt; ++t)
        if (r[t] && d->terms[t].op == TH_TERM_STAT)
          TH_REQUIRE(d->outputs[o].full == 0 || d->folds[d->terms[t].ref].scan != TH_SCAN_NONE,
                     "th_build_floor: output " + std::to_string(o) + " reads a plain fold's result at a position");
    }
    // Where the memory terms run along the first scanned axis, a workgroup
    // per item scans its positions in parallel (chunks of 256 lanes, four
    // positions a lane going forward); else a thread per item, items side by
    // side, each sweeping in order.
    int pos_unit = 0, item_unit = 0;
    const int s0 = pl.swept[0], k0 = pl.kept.empty() ? -1 : pl.kept[0];
    auto score = [&](const th_affine& a) {
      if (std::llabs(a.coeff[s0]) == 1 && pl.E[s0] > 1) ++pos_unit;
      else if (k0 >= 0 && std::llabs(a.coeff[k0]) == 1 && pl.E[k0] > 1) ++item_unit;
    };
    for (int t = 0; t < nt; ++t)
      if (d->terms[t].op == TH_TERM_LOAD && pl.dep[t]) score(d->terms[t].index);
    for (int o = 0; o < d->n_outputs; ++o)
      if (d->outputs[o].full) score(d->outputs[o].index);
    pl.rows = pl.count >= 64 && (pl.kept.empty() || pos_unit > item_unit);
    if (pl.rows) {
      pl.S = 1;
      pl.L = 256;
      pl.P = 1;
      pl.W = (!pl.reverse && !pl.gathers && pl.E[s0] % 4 == 0 && pl.count >= 256) ? 4 : 1;
      pl.vax = pl.W > 1 ? s0 : -1;
      pl.qn = pl.count / pl.W;
    } else {
      pl.S = 256;
      pl.L = pl.P = pl.W = 1;
      pl.qn = pl.count;
    }
  } else if (pl.reduction) {
    for (int f = 0; f < d->n_folds; ++f)
      if (d->folds[f].phase >= 1) pl.phases.push_back(d->folds[f].phase);
    std::sort(pl.phases.begin(), pl.phases.end());
    pl.phases.erase(std::unique(pl.phases.begin(), pl.phases.end()), pl.phases.end());
    for (int f = 0; f < d->n_folds; ++f) {
      if (d->folds[f].phase == 0) continue;
      std::vector<int> roots{d->folds[f].body};
      if (d->folds[f].weight >= 0) roots.push_back(d->folds[f].weight);
      TH_REQUIRE(max_stat_phase(d, reach(d, roots)) < d->folds[f].phase,
                 "th_build_floor: fold " + std::to_string(f) + " reads a statistic of its own or a later phase");
    }
    // Rows or columns: where the memory terms' unit strides point.
    int pos_unit = 0, item_unit = 0;
    const int s0 = pl.swept[0], k0 = pl.kept.empty() ? -1 : pl.kept[0];
    auto score = [&](const th_affine& a) {
      if (std::llabs(a.coeff[s0]) == 1 && pl.E[s0] > 1) ++pos_unit;
      else if (k0 >= 0 && std::llabs(a.coeff[k0]) == 1 && pl.E[k0] > 1) ++item_unit;
    };
    for (int t = 0; t < nt; ++t)
      if (d->terms[t].op == TH_TERM_LOAD && pl.dep[t]) score(d->terms[t].index);
    for (int o = 0; o < d->n_outputs; ++o)
      if (d->outputs[o].full) score(d->outputs[o].index);
    pl.rows = pl.kept.empty() || pos_unit >= item_unit;
    if (pl.rows) {
      pl.S = 1;
      pl.W = (pl.E[s0] % 4 == 0 && pl.count >= 256 && !pl.gathers) ? 4 : 1;
      pl.vax = pl.W > 1 ? s0 : -1;
      pl.qn = pl.count / pl.W;
      pl.L = (int)std::min<int64_t>(256, std::max<int64_t>(64, nextpow2(pl.qn)));
      // Split an item's positions among workgroups only when few items leave
      // the device idle and each lane would otherwise sweep 64+ steps: a
      // shorter fold costs less than the extra launch and merge (one
      // workgroup's 128 dependent steps over 128 K floats take ~32 us, the
      // same fold in 16 parts and a merge a few).
      if (pl.items < 8 * kCUs && pl.qn >= (int64_t)pl.L * 64) {
        int64_t want = (8 * kCUs + pl.items - 1) / std::max<int64_t>(pl.items, 1);
        want = std::min<int64_t>(want, pl.qn / ((int64_t)pl.L * 8));
        pl.P = (int)std::max<int64_t>(1, std::min<int64_t>(want, 1024));
      }
    } else {
      pl.S = 64;
      pl.W = 1;
      pl.qn = pl.count;
      int64_t want = (int64_t)kCUs * 1024 / std::max<int64_t>(pl.items, 1);
      want = std::max<int64_t>(1, std::min<int64_t>(want, pl.qn / 8));
      pl.L = (int)std::min<int64_t>(4, prevpow2(want));
      pl.P = (int)std::max<int64_t>(1, std::min<int64_t>(want / pl.L, 1024));
    }
    // Loads kept in registers across the phases when an item's share fits.
    if (pl.P == 1 && !pl.gathers) {
      int64_t iters = (pl.qn + pl.L - 1) / pl.L;
      int cached = 0;
      for (int t = 0; t < nt; ++t) cached += d->terms[t].op == TH_TERM_LOAD && pl.dep[t];
      if (iters >= 1 && iters <= kMaxIters && cached * iters * pl.W <= kResidentFloats) {
        pl.resident = true;
        pl.iters = (int)iters;
      }
    }
  } else if (pl.recurrence) {
    // A thread per position of the parallel axes, stepping in order.
    pl.kept.clear();
    pl.swept.clear();
    for (int k = 0; k < pl.rank; ++k) ((d->reduced >> k & 1) ? pl.swept : pl.kept).push_back(k);
    pl.items = 1;
    for (int k : pl.kept) pl.items *= pl.E[k];
    pl.W = 1;
    pl.qn = pl.items;
    pl.S = 256;
    pl.L = 1;
  } else {
    pl.kept.clear();
    for (int k = 0; k < pl.rank; ++k) pl.kept.push_back(k);
    pl.items = 1;
    for (int k = 0; k < pl.rank; ++k) pl.items *= pl.E[k];
    pl.W = (pl.E[0] % 4 == 0 && pl.E[0] >= 4 && !pl.gathers && !pl.ordered) ? 4 : 1;
    pl.vax = pl.W > 1 ? 0 : -1;
    pl.qn = pl.items / pl.W;
    // In order: one wave whose first lane takes every item in turn.
    pl.S = pl.ordered ? 64 : 256;
    pl.L = 1;
  }
  // Vector accesses: aligned pointer, and every other coefficient and the
  // constant multiples of 4 (the W positions start at multiples of 4).
  pl.vec_ok.assign(d->n_values, 0);
  if (pl.W > 1) {
    for (int v = 0; v < d->n_values; ++v) {
      const th_floor_value& x = d->values[v];
      uintptr_t need = x.dtype == TH_F32 ? 16 : 8;
      pl.vec_ok[v] = ((uintptr_t)x.ptr % need) == 0;
    }
  }
  return TH_OK;
}

bool vector_access(const Plan& pl, int value, const th_affine& a) {
  if (pl.W == 1 || !pl.vec_ok[value] || a.coeff[pl.vax] != 1) return false;
  if (a.constant % 4 != 0) return false;
  for (int k = 0; k < pl.rank; ++k)
    if (k != pl.vax && pl.E[k] > 1 && a.coeff[k] % 4 != 0) return false;
  return true;
}

std::string affine(const Plan& pl, const th_affine& a) {
  std::ostringstream s;
  s << "(" << a.constant << "L";
  for (int k = 0; k < kRank; ++k)
    if (a.coeff[k] != 0 && (k >= pl.rank || pl.E[k] > 1)) s << " + " << a.coeff[k] << "L * i" << k;
  for (const th_part& q : a.part) {
    if (q.kind == TH_PART_NONE || q.coeff == 0) continue;
    std::ostringstream in;
    in << "(" << q.constant << "L";
    for (int k = 0; k < pl.rank; ++k)
      if (q.inner[k] != 0 && pl.E[k] > 1) in << " + " << q.inner[k] << "L * i" << k;
    in << ")";
    int64_t lo, hi;
    span(q.constant, q.inner, pl.E, pl.rank, lo, hi);
    s << " + " << q.coeff << "L * ";
    if (lo >= 0)  // never negative: C's / and % are the floor division and remainder
      s << "(" << in.str() << (q.kind == TH_PART_DIV ? " / " : " % ") << q.divisor << "L)";
    else
      s << (q.kind == TH_PART_DIV ? "th_fld(" : "th_fmod(") << in.str() << ", " << q.divisor << "L)";
  }
  s << ")";
  return s.str();
}

std::string stat_name(int f, int obs) { return "st" + std::to_string(f) + "_" + std::to_string(obs); }

// ---- source -----------------------------------------------------------------

const char* kPrelude = R"(typedef unsigned short th_bf16;
__device__ __forceinline__ float th_bf(th_bf16 h) { return __builtin_bit_cast(float, ((unsigned)h) << 16); }
__device__ __forceinline__ th_bf16 th_tobf(float f) {
  unsigned u = __builtin_bit_cast(unsigned, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (th_bf16)0x7fc0u;
  return (th_bf16)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float th_ld(const float* p, long i) { return p[i]; }
__device__ __forceinline__ float th_ld(const th_bf16* p, long i) { return th_bf(p[i]); }
__device__ __forceinline__ float th_ld(float* p, long i) { return p[i]; }
__device__ __forceinline__ float th_ld(th_bf16* p, long i) { return th_bf(p[i]); }
// An integer value read as a term (a seed, a count): its fp32 value.
__device__ __forceinline__ float th_ld(const int* p, long i) { return (float)p[i]; }
__device__ __forceinline__ float th_ld(const long* p, long i) { return (float)p[i]; }
__device__ __forceinline__ float th_ld(int* p, long i) { return (float)p[i]; }
__device__ __forceinline__ float th_ld(long* p, long i) { return (float)p[i]; }
__device__ __forceinline__ float th_ldn(const float* p, long i) { return __builtin_nontemporal_load(p + i); }
__device__ __forceinline__ float th_ldn(const th_bf16* p, long i) { return th_bf(__builtin_nontemporal_load(p + i)); }
__device__ __forceinline__ float th_ldn(float* p, long i) { return th_ldn((const float*)p, i); }
__device__ __forceinline__ float th_ldn(th_bf16* p, long i) { return th_ldn((const th_bf16*)p, i); }
__device__ __forceinline__ void th_st(float* p, long i, float v) { p[i] = v; }
__device__ __forceinline__ void th_st(th_bf16* p, long i, float v) { p[i] = th_tobf(v); }
__device__ __forceinline__ void th_stn(float* p, long i, float v) { __builtin_nontemporal_store(v, p + i); }
__device__ __forceinline__ void th_stn(th_bf16* p, long i, float v) { __builtin_nontemporal_store(th_tobf(v), p + i); }
__device__ __forceinline__ long th_ldi(const int* p, long i) { return (long)p[i]; }
__device__ __forceinline__ long th_ldi(const long* p, long i) { return p[i]; }
// A gathered position, held inside its value (0 .. n - 1).
__device__ __forceinline__ long th_clampi(long i, long n) { return i < 0 ? 0 : (i >= n ? n - 1 : i); }
// Floor division by a positive d, and the remainder in 0 .. d - 1 (Div and Mod atoms).
__device__ __forceinline__ long th_fld(long x, long d) { return x >= 0 ? x / d : -((-x + d - 1) / d); }
__device__ __forceinline__ long th_fmod(long x, long d) { return x - d * th_fld(x, d); }
__device__ __forceinline__ void th_add(float* p, long i, float v) { atomicAdd(p + i, v); }
// In order (one thread): the elements add in the items' order, every run alike.
__device__ __forceinline__ void th_add_ordered(float* p, long i, float v) { p[i] = p[i] + v; }
__device__ __forceinline__ float th_abs(float x) { return fabsf(x); }
__device__ __forceinline__ float th_abs2(float x) { return x * x; }
__device__ __forceinline__ float th_sqrt(float x) { return sqrtf(x); }
// exp(x) = 2^h 2^l, h = x log2(e) rounded, l its rounding error (an fma)
// plus the tail of log2(e); 2^l = 1 + l ln 2 to second order.  About 2 ulp
// against 13 instructions of the library's expf; x = -inf, +inf and NaN give
// 0, inf and NaN (l is then NaN, and fminf takes the 1).
__device__ __forceinline__ float th_exp(float x) {
  const float h = x * 0x1.715476p+0f;
  const float l = fmaf(x, 0x1.4ae0bep-26f, fmaf(x, 0x1.715476p+0f, -h));
  const float e = __builtin_amdgcn_exp2f(h);
  return fmaf(e, fminf(l * 0x1.62e430p-1f, 1.0f), e);
}
__device__ __forceinline__ float th_log(float x) { return logf(x); }
__device__ __forceinline__ float th_tanh(float x) { return tanhf(x); }
__device__ __forceinline__ float th_sin(float x) { return sinf(x); }
__device__ __forceinline__ float th_cos(float x) { return cosf(x); }
__device__ __forceinline__ float th_log1p(float x) { return log1pf(x); }
__device__ __forceinline__ float th_expm1(float x) { return expm1f(x); }
__device__ __forceinline__ float th_pow(float x, float y) { return powf(x, y); }
__device__ __forceinline__ float th_max(float x, float y) { return fmaxf(x, y); }
__device__ __forceinline__ float th_min(float x, float y) { return fminf(x, y); }
__device__ __forceinline__ float th_lt(float x, float y) { return x < y ? 1.0f : 0.0f; }
__device__ __forceinline__ float th_le(float x, float y) { return x <= y ? 1.0f : 0.0f; }
__device__ __forceinline__ float th_gt(float x, float y) { return x > y ? 1.0f : 0.0f; }
__device__ __forceinline__ float th_ge(float x, float y) { return x >= y ? 1.0f : 0.0f; }
__device__ __forceinline__ float th_eq(float x, float y) { return x == y ? 1.0f : 0.0f; }
__device__ __forceinline__ float th_ne(float x, float y) { return x != y ? 1.0f : 0.0f; }
__device__ __forceinline__ float th_ifelse(float c, float a, float b) { return c != 0.0f ? a : b; }
__device__ __forceinline__ float th_round(float x) { return rintf(x); }
__device__ __forceinline__ float th_floor(float x) { return floorf(x); }
__device__ __forceinline__ float th_ceil(float x) { return ceilf(x); }
__device__ __forceinline__ float th_sign(float x) { return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : x); }
__device__ __forceinline__ float th_clamp(float x, float lo, float hi) { return x > hi ? hi : (x < lo ? lo : x); }
__device__ __forceinline__ float th_fma(float a, float b, float c) { return fmaf(a, b, c); }
__device__ __forceinline__ float th_inv(float x) { return 1.0f / x; }
// Cast{BFloat16}: rounded to bfloat16, then widened back to fp32.
__device__ __forceinline__ float th_rbf(float x) { return th_bf(th_tobf(x)); }
// The dropout fixture's keep scale (test/fixtures/operations.jl:88-103,
// stream 0): the key and the 1-based position (integers held exactly in
// fp32) hashed in wrapping 32-bit arithmetic with logical shifts; the top 24
// bits as a fraction u, kept at scale 1 / (1 - rate) when u >= rate.
__device__ __forceinline__ float th_dropout(float key, float pos, float rate) {
  unsigned h = (unsigned)(int)key * 0x9e3779b1u ^ (unsigned)(int)pos * 0xc2b2ae35u;
  h ^= h >> 16;
  h *= 0x7feb352du;
  h ^= h >> 15;
  h *= 0x846ca68bu;
  h ^= h >> 16;
  const float u = (float)(h >> 8) * 0x1p-24f;
  return u >= rate ? 1.0f / (1.0f - rate) : 0.0f;
}
// lse_shift (src/Compiler/IR/folds.jl:194): the maximum when finite, else 0.
__device__ __forceinline__ float th_shift(float m) { return __builtin_isfinite(m) ? m : 0.0f; }
// Relative{Exponential}: state (m, s), s the weighted sum of exp(y - shift(m)).
// One exponential a step: the smaller of m and y is rebased to the larger.
__device__ __forceinline__ void th_exp_step(float& m, float& s, float y, float g) {
  const float n = fmaxf(m, y);
  const float e = th_exp(fminf(m, y) - th_shift(n));
  s = (y > m) ? s * e + g : s + g * e;
  m = n;
}
__device__ __forceinline__ void th_exp_comb(float& m, float& s, float m2, float s2) {
  const float n = fmaxf(m, m2);
  const float h = th_shift(n);
  s = s * th_exp(m - h) + s2 * th_exp(m2 - h);
  m = n;
}
// The linear recurrence h = a h' + b: state (product of the a's, h).
__device__ __forceinline__ void th_lin_step(float& p, float& h, float a, float b) { p *= a; h = fmaf(a, h, b); }
__device__ __forceinline__ void th_lin_comb(float& p, float& h, float p2, float h2) { h = fmaf(p2, h, h2); p *= p2; }
// The extreme and where it is: state (y, i).  Base's isless (NaN the
// largest, -0.0 before 0.0) for findmax, its isgreater (NaN the smallest) for
// findmin, in comparisons alone; the smaller index among equals.
__device__ __forceinline__ bool th_lesser(float x, float y) {
  return x != x ? false : ((y != y) || x < y || (x == y && 1.0f / x < 1.0f / y));
}
__device__ __forceinline__ bool th_greater(float x, float y) {
  return x != x ? false : ((y != y) || y < x || (x == y && 1.0f / y < 1.0f / x));
}
__device__ __forceinline__ void th_amax_comb(float& y, float& i, float y2, float i2) {
  const bool t = th_lesser(y, y2) || (!th_lesser(y2, y) && i2 < i);
  y = t ? y2 : y;
  i = t ? i2 : i;
}
__device__ __forceinline__ void th_amin_comb(float& y, float& i, float y2, float i2) {
  const bool t = th_greater(y, y2) || (!th_greater(y2, y) && i2 < i);
  y = t ? y2 : y;
  i = t ? i2 : i;
}
// Relative{Square}: state (n, mean, squared deviations), Welford's step and
// Chan's combination.
__device__ __forceinline__ void th_sq_step(float& n, float& a, float& q, float y) {
  n += 1.0f;
  const float e = y - a;
  a += e / n;
  q += e * (y - a);
}
__device__ __forceinline__ void th_sq_comb(float& n, float& a, float& q, float n2, float a2, float q2) {
  if (n2 == 0.0f) return;
  if (n == 0.0f) { n = n2; a = a2; q = q2; return; }
  const float t = n + n2;
  const float e = a2 - a;
  a += e * (n2 / t);
  q += q2 + e * e * (n * (n2 / t));
  n = t;
}
)";

const char* kVector = R"(typedef float th_v __attribute__((ext_vector_type(4)));
typedef unsigned short th_h4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ th_v th_splat(float x) { return (th_v){x, x, x, x}; }
__device__ __forceinline__ th_v th_iota() { return (th_v){0.0f, 1.0f, 2.0f, 3.0f}; }
__device__ __forceinline__ th_v th_ld4(const float* p, long i) { return *(const th_v*)(p + i); }
__device__ __forceinline__ th_v th_ld4(const th_bf16* p, long i) {
  const th_h4 h = *(const th_h4*)(p + i);
  return (th_v){th_bf(h[0]), th_bf(h[1]), th_bf(h[2]), th_bf(h[3])};
}
__device__ __forceinline__ th_v th_ld4n(const float* p, long i) { return __builtin_nontemporal_load((const th_v*)(p + i)); }
__device__ __forceinline__ th_v th_ld4n(const th_bf16* p, long i) {
  const th_h4 h = __builtin_nontemporal_load((const th_h4*)(p + i));
  return (th_v){th_bf(h[0]), th_bf(h[1]), th_bf(h[2]), th_bf(h[3])};
}
__device__ __forceinline__ th_v th_ld4n(float* p, long i) { return th_ld4n((const float*)p, i); }
__device__ __forceinline__ th_v th_ld4n(th_bf16* p, long i) { return th_ld4n((const th_bf16*)p, i); }
__device__ __forceinline__ th_v th_ld4(float* p, long i) { return th_ld4((const float*)p, i); }
__device__ __forceinline__ th_v th_ld4(th_bf16* p, long i) { return th_ld4((const th_bf16*)p, i); }
template <class T> __device__ __forceinline__ th_v th_lds4(T p, long i, long s) {
  return (th_v){th_ld(p, i), th_ld(p, i + s), th_ld(p, i + 2 * s), th_ld(p, i + 3 * s)};
}
__device__ __forceinline__ void th_st4(float* p, long i, th_v v) { *(th_v*)(p + i) = v; }
__device__ __forceinline__ void th_st4(th_bf16* p, long i, th_v v) {
  *(th_h4*)(p + i) = (th_h4){th_tobf(v[0]), th_tobf(v[1]), th_tobf(v[2]), th_tobf(v[3])};
}
__device__ __forceinline__ void th_st4n(float* p, long i, th_v v) { __builtin_nontemporal_store(v, (th_v*)(p + i)); }
__device__ __forceinline__ void th_st4n(th_bf16* p, long i, th_v v) {
  __builtin_nontemporal_store((th_h4){th_tobf(v[0]), th_tobf(v[1]), th_tobf(v[2]), th_tobf(v[3])}, (th_h4*)(p + i));
}
template <class T> __device__ __forceinline__ void th_sts4(T p, long i, long s, th_v v) {
  th_st(p, i, v[0]); th_st(p, i + s, v[1]); th_st(p, i + 2 * s, v[2]); th_st(p, i + 3 * s, v[3]);
}
#define TH_V1(f) __device__ __forceinline__ th_v f(th_v x) { return (th_v){f(x[0]), f(x[1]), f(x[2]), f(x[3])}; }
#define TH_V2(f) __device__ __forceinline__ th_v f(th_v x, th_v y) { \
  return (th_v){f(x[0], y[0]), f(x[1], y[1]), f(x[2], y[2]), f(x[3], y[3])}; }
#define TH_V3(f) __device__ __forceinline__ th_v f(th_v x, th_v y, th_v z) { \
  return (th_v){f(x[0], y[0], z[0]), f(x[1], y[1], z[1]), f(x[2], y[2], z[2]), f(x[3], y[3], z[3])}; }
TH_V1(th_abs) TH_V1(th_abs2) TH_V1(th_sqrt) TH_V1(th_exp) TH_V1(th_log) TH_V1(th_tanh) TH_V1(th_sin)
TH_V1(th_cos) TH_V1(th_log1p) TH_V1(th_expm1) TH_V1(th_round) TH_V1(th_floor) TH_V1(th_ceil)
TH_V1(th_sign) TH_V1(th_inv) TH_V1(th_rbf)
TH_V2(th_pow) TH_V2(th_max) TH_V2(th_min) TH_V2(th_lt) TH_V2(th_le) TH_V2(th_gt) TH_V2(th_ge)
TH_V2(th_eq) TH_V2(th_ne)
TH_V3(th_ifelse) TH_V3(th_clamp) TH_V3(th_fma) TH_V3(th_dropout)
__device__ __forceinline__ void th_exp_step(th_v& m, th_v& s, th_v y, th_v g) {
#pragma unroll
  for (int j = 0; j < 4; ++j) { float a = m[j], b = s[j]; th_exp_step(a, b, y[j], g[j]); m[j] = a; s[j] = b; }
}
__device__ __forceinline__ void th_lin_step(th_v& p, th_v& h, th_v a, th_v b) { p *= a; h = a * h + b; }
__device__ __forceinline__ void th_amax_comb(th_v& y, th_v& i, th_v y2, th_v i2) {
#pragma unroll
  for (int j = 0; j < 4; ++j) { float a = y[j], b = i[j]; th_amax_comb(a, b, y2[j], i2[j]); y[j] = a; i[j] = b; }
}
__device__ __forceinline__ void th_amin_comb(th_v& y, th_v& i, th_v y2, th_v i2) {
#pragma unroll
  for (int j = 0; j < 4; ++j) { float a = y[j], b = i[j]; th_amin_comb(a, b, y2[j], i2[j]); y[j] = a; i[j] = b; }
}
__device__ __forceinline__ void th_sq_step(th_v& n, th_v& a, th_v& q, th_v y) {
#pragma unroll
  for (int j = 0; j < 4; ++j) { float x = n[j], b = a[j], c = q[j]; th_sq_step(x, b, c, y[j]); n[j] = x; a[j] = b; q[j] = c; }
}
)";

const char* kScalar = R"(typedef float th_v;
__device__ __forceinline__ float th_splat(float x) { return x; }
)";

struct Stage {
  std::string name;
  int phase_index;  // the phase a split stage folds; -1 for the stage that stores
};

// What decides a code object beside its source and options: the hiprtc that
// compiles it, the HIP runtime that loads it, and the layout of this store.
// It is written into every generated source, so the store's key (a hash of
// the source) changes with it and entries of another toolchain are never read.
const int kStoreSchema = 2;

std::string toolchain() {
  static const std::string s = [] {
    int major = 0, minor = 0, runtime = 0;
    hiprtcVersion(&major, &minor);
    if (hipRuntimeGetVersion(&runtime) != hipSuccess) runtime = HIP_VERSION;
    return "hiprtc " + std::to_string(major) + "." + std::to_string(minor) + ", HIP runtime " +
           std::to_string(runtime) + ", store schema " + std::to_string(kStoreSchema);
  }();
  return s;
}

class Writer {
 public:
  explicit Writer(const Plan& pl) : pl_(pl), d_(pl.d) {}

  std::string source(std::vector<Stage>& stages, const std::string& base) {
    std::ostringstream& o = o_;
    o << "// tempest-hip floor: " << describe() << "\n";
    o << "// toolchain: " << toolchain() << "\n";
    o << kPrelude << (pl_.W > 1 ? kVector : kScalar);
    o << "struct th_args { void* p[" << (d_->n_values + (pl_.reduction ? d_->n_folds : 0)) << "]; };\n";
    if (pl_.recurrence) {
      stages.push_back({base + "_0", -1});
      recurrence(stages.back().name);
    } else if (!pl_.reduction) {
      stages.push_back({base + "_0", -1});
      pointwise(stages.back().name);
    } else if (pl_.scan) {
      stages.push_back({base + "_0", -1});
      scan(stages.back().name);
    } else if (pl_.P == 1) {
      stages.push_back({base + "_0", -1});
      reduction(stages.back().name, -1);
    } else {
      for (size_t j = 0; j < pl_.phases.size(); ++j) {
        stages.push_back({base + "_" + std::to_string(j), (int)j});
        reduction(stages.back().name, (int)j);
      }
      stages.push_back({base + "_" + std::to_string(pl_.phases.size()), -1});
      reduction(stages.back().name, -1);
    }
    return o.str();
  }

  std::string describe() const {
    std::ostringstream s;
    if (pl_.recurrence) {
      s << "recurrence, " << pl_.items << " items stepping " << pl_.E[pl_.step] << " positions of axis " << pl_.step
        << (pl_.reverse ? ", reversed" : "");
    } else if (!pl_.reduction) {
      s << "pointwise, " << pl_.items << " positions, width " << pl_.W;
    } else if (pl_.scan) {
      s << "scan, " << pl_.items << " items of " << pl_.count << " positions, "
        << (pl_.rows ? "a workgroup per item, width " + std::to_string(pl_.W) : std::string("a thread per item"))
        << (pl_.reverse ? ", reversed" : "");
    } else {
      s << (pl_.rows ? "rows" : "columns") << ", " << pl_.items << " items of " << pl_.count
        << " positions, side " << pl_.S << ", lanes " << pl_.L << ", parts " << pl_.P << ", width " << pl_.W
        << ", " << pl_.phases.size() << " phase(s), "
        << (pl_.resident ? "resident (" + std::to_string(pl_.iters) + " steps)" : std::string("streamed"));
    }
    return s.str();
  }

 private:
  const Plan& pl_;
  const th_floor_desc* d_;
  std::ostringstream o_;
  int uid_ = 0;
  bool stat_vec_ = false;  // scan results read per position (the parallel scan)

  std::string vtype(int v) const {
    switch (d_->values[v].dtype) {
      case TH_F32: return "float";
      case TH_BF16: return "th_bf16";
      case TH_I32: return "int";
      default: return "long";
    }
  }
  // The long variable each emitted integer load lives in (the latest scope's).
  std::map<int, std::string> gvar_;
  // An address: the affine part, plus the gathered term's value, clamped.
  std::string addr(const th_affine& a, int value) {
    std::string e = affine(pl_, a);
    if (a.gather < 0) return e;
    return "th_clampi(" + e + " + " + std::to_string(a.gather_coeff) + "L * " + gvar_.at(a.gather) + ", " +
           std::to_string(d_->values[value].length) + "L)";
  }
  std::string vname(int v) const { return "v" + std::to_string(v); }
  // An output's term, and the term its address gathers by.
  void out_roots(std::vector<int>& roots, int x) const {
    roots.push_back(d_->outputs[x].term);
    if (d_->outputs[x].index.gather >= 0) roots.push_back(d_->outputs[x].index.gather);
  }

  void header(const std::string& name) {
    std::ostringstream& o = o_;
    const int nt = pl_.S * pl_.L;
    o << "extern \"C\" __global__ __launch_bounds__(" << nt << ") void " << name << "(const th_args a) {\n";
    for (int v = 0; v < d_->n_values; ++v) {
      bool ro = !pl_.written[v];
      o << "  " << (ro ? "const " : "") << vtype(v) << "* " << (ro ? "__restrict__ " : "") << vname(v)
        << " = (" << (ro ? "const " : "") << vtype(v) << "*)a.p[" << v << "];\n";
    }
    o << "  long i0 = 0, i1 = 0, i2 = 0, i3 = 0;\n";
    o << "  (void)i0; (void)i1; (void)i2; (void)i3;\n";
  }

  // The value of term t in a scope: `vec` gives th_v values, `cached` reads
  // the swept loads from their registers (index `it`).
  std::string term_expr(int t, bool vec, bool cached, const std::map<int, std::string>& names,
                        bool nt = false) {
    const th_term& m = d_->terms[t];
    const std::string n = nt ? "n" : "";
    auto arg = [&](int j) { return names.at(m.args[j]); };
    switch (m.op) {
      case TH_TERM_LOAD: {
        if (cached && pl_.dep[t]) return "c" + std::to_string(t) + "[it]";
        std::string p = vname(m.ref), at = addr(m.index, m.ref);
        if (is_int(d_->values[m.ref].dtype)) return "th_ldi(" + p + ", " + at + ")";
        if (!vec || pl_.W == 1) return "th_ld" + n + "(" + p + ", " + at + ")";
        const int64_t cv = m.index.coeff[pl_.vax];
        if (cv == 0) return "th_splat(th_ld(" + p + ", " + at + "))";
        if (vector_access(pl_, m.ref, m.index)) return "th_ld4" + n + "(" + p + ", " + at + ")";
        return "th_lds4(" + p + ", " + at + ", " + std::to_string(cv) + "L)";
      }
      case TH_TERM_LIT:
        return vec ? "th_splat(" + flt(m.lit) + ")" : flt(m.lit);
      case TH_TERM_INDEX: {
        std::string x = "(float)" + affine(pl_, m.index);
        if (!vec || pl_.W == 1) return vec ? "th_splat(" + x + ")" : x;
        const int64_t cv = m.index.coeff[pl_.vax];
        if (cv == 0) return "th_splat(" + x + ")";
        return "(th_splat(" + x + ") + " + flt((float)cv) + " * th_iota())";
      }
      case TH_TERM_STAT: {
        if (stat_vec_ && d_->folds[m.ref].scan != TH_SCAN_NONE)
          return "s" + stat_name(m.ref, m.observe);  // this lane's positions
        std::string s = stat_name(m.ref, m.observe);
        return vec ? "th_splat(" + s + ")" : s;
      }
      default:
        break;
    }
    switch (m.fn) {
      case TH_FN_ADD: return "(" + arg(0) + " + " + arg(1) + ")";
      case TH_FN_SUB: return "(" + arg(0) + " - " + arg(1) + ")";
      case TH_FN_MUL: return "(" + arg(0) + " * " + arg(1) + ")";
      case TH_FN_DIV: return "(" + arg(0) + " / " + arg(1) + ")";
      case TH_FN_NEG: return "(-" + arg(0) + ")";
      default: break;
    }
    std::string s = std::string(fn_name(m.fn)) + "(";
    for (int j = 0; j < arity(m.fn); ++j) s += (j ? ", " : "") + arg(j);
    return s + ")";
  }

  // Emit the terms of `want`, in order, as named values of this scope.
  void emit(const std::string& ind, const std::vector<char>& want, bool vec, bool cached,
            std::map<int, std::string>& names, const std::map<int, std::string>* outer) {
    const std::string ty = vec ? "th_v" : "float";
    for (int t = 0; t < d_->n_terms; ++t) {
      if (!want[t] || names.count(t)) continue;
      // Arguments computed outside the scope, as scalars: splat them here.
      if (d_->terms[t].op == TH_TERM_APPLY && outer) {
        for (int j = 0; j < arity(d_->terms[t].fn); ++j) {
          int u = d_->terms[t].args[j];
          if (!names.count(u) && outer->count(u))
            names[u] = vec ? "th_splat(" + outer->at(u) + ")" : outer->at(u);
        }
      }
      std::string n = "t" + std::to_string(uid_++);
      const th_term& m = d_->terms[t];
      if (m.op == TH_TERM_RECOMPUTE) {
        recompute(ind, t, n);
        names[t] = vec ? "th_splat(" + n + ")" : n;
        continue;
      }
      if (m.op == TH_TERM_LOAD && is_int(d_->values[m.ref].dtype)) {
        // An integer: kept as such for the addresses that gather by it.
        o_ << ind << "const long " << n << " = " << term_expr(t, false, false, names) << ";\n";
        gvar_[t] = n;
        names[t] = vec ? "th_splat((float)" + n + ")" : "(float)" + n;
        continue;
      }
      o_ << ind << "const " << ty << " " << n << " = " << term_expr(t, vec, cached, names) << ";\n";
      names[t] = n;
      // A float load an address gathers by (groups that gather run at width 1).
      if (m.op == TH_TERM_LOAD && !vec) gvar_[t] = "((long)" + n + ")";
    }
  }

  // A fold computed where it is read (Recomputed, codegen/scalar.jl:88-110):
  // a loop over its own axes (positions rank, rank + 1, ...), its body
  // computed afresh at each, then the observation read into `n`.
  void recompute(const std::string& ind, int t, const std::string& n) {
    const th_term& m = d_->terms[t];
    const th_fold& f = d_->folds[m.ref];
    const int K = state_size(f.kind);
    const std::string base = "r" + std::to_string(uid_++), j = "j" + base;
    std::vector<std::string> c = comps(base, K);
    for (int k = 0; k < K; ++k) o_ << ind << "float " << c[k] << " = " << identity(f.kind, k) << ";\n";
    int64_t count = 1;
    for (int q = 0; q < f.n_inner; ++q) count *= f.inner[q];
    o_ << ind << "for (long " << j << " = 0; " << j << " < " << count << "L; ++" << j << ") {\n";
    const std::string in = ind + "  ";
    o_ << in << "long r = " << j << ";\n";
    for (int q = 0; q < f.n_inner; ++q) {
      const int k = pl_.rank + q;
      if (q + 1 == f.n_inner) o_ << in << "i" << k << " = r;\n";
      else o_ << in << "i" << k << " = r % " << f.inner[q] << "L; r /= " << f.inner[q] << "L;\n";
    }
    std::vector<int> roots{f.body};
    if (f.weight >= 0) roots.push_back(f.weight);
    std::map<int, std::string> inner;
    const std::map<int, std::string> saved = gvar_;
    emit(in, reach(d_, roots), false, false, inner, nullptr);
    o_ << in << step_stmt(f.kind, c, inner.at(f.body), f.weight >= 0 ? inner.at(f.weight) : std::string("1.0f"))
       << "\n";
    gvar_ = saved;
    o_ << ind << "}\n";
    o_ << ind << "const float " << n << " = " << observe_expr(f.kind, m.observe, c) << ";\n";
  }

  // A recurrence (recurrence_kernel, codegen/scalar.jl:402-440): a thread per
  // position of the parallel axes steps along the step axis; at each step the
  // outputs run in order, each over the other reduced axes its address
  // mentions, reading what the steps so far stored (plain loads and stores:
  // a thread reads its own writes).
  void recurrence(const std::string& name) {
    std::ostringstream& o = o_;
    header(name);
    const int sa = pl_.step;
    const int64_t E = pl_.E[sa];
    o << "  const long item = (long)blockIdx.x * " << pl_.S << " + threadIdx.x;\n";
    o << "  if (item >= " << pl_.items << "L) return;\n";
    delinearize("  ", "item", pl_.kept);
    o << "  for (long s = 0; s < " << E << "L; ++s) {\n";
    o << "    i" << sa << " = " << (pl_.reverse ? std::to_string(E - 1) + "L - s" : std::string("s")) << ";\n";
    for (int x = 0; x < d_->n_outputs; ++x) {
      const th_output& out = d_->outputs[x];
      const char* when = out.full == TH_STEP_FIRST ? "s == 0L" : out.full == TH_STEP_LAST ? "s == LASTL"
                         : out.full == TH_STEP_CARRY ? "s != LASTL" : "true";
      std::string cond = when;
      const size_t at = cond.find("LAST");
      if (at != std::string::npos) cond.replace(at, 4, std::to_string(E - 1));
      std::vector<int> inner;
      for (int k : pl_.swept) {
        if (k == sa) continue;
        bool mentioned = out.index.coeff[k] != 0;
        for (const th_part& q : out.index.part) mentioned |= q.kind != TH_PART_NONE && q.coeff != 0 && q.inner[k] != 0;
        if (mentioned) inner.push_back(k);
      }
      int64_t count = 1;
      for (int k : inner) count *= pl_.E[k];
      o << "    if (" << cond << ") {  // output " << x << "\n";
      for (int k : pl_.swept)
        if (k != sa) o << "      i" << k << " = 0;\n";
      o << "      for (long p = 0; p < " << count << "L; ++p) {\n";
      delinearize("        ", "p", inner);
      std::vector<int> roots;
      out_roots(roots, x);
      std::map<int, std::string> names;
      emit("        ", reach(d_, roots), false, false, names, nullptr);
      th_output plain = out;
      plain.full = 0;
      store("        ", plain, names.at(out.term), false);
      o << "      }\n    }\n";
    }
    o << "  }\n}\n";
  }

  // Hoisted terms (not moving along the sweep) then swept ones.
  void split_emit(const std::string& ind_out, const std::vector<char>& r, std::map<int, std::string>& hoisted) {
    std::vector<char> h(d_->n_terms, 0);
    for (int t = 0; t < d_->n_terms; ++t) h[t] = r[t] && !pl_.dep[t];
    emit(ind_out, h, false, false, hoisted, nullptr);
  }

  std::string name_of(int t, const std::map<int, std::string>& inner, const std::map<int, std::string>& hoisted, bool vec) {
    if (inner.count(t)) return inner.at(t);
    return vec ? "th_splat(" + hoisted.at(t) + ")" : hoisted.at(t);
  }

  // The sweep over an item's positions, this thread's share.  `body` writes
  // the statements at one step of W positions.
  template <class Body>
  void sweep(const std::string& ind, bool split_parts, Body body) {
    std::ostringstream& o = o_;
    const bool guard_live = pl_.items % pl_.S != 0;
    const std::string qn = std::to_string(pl_.qn) + "L";
    if (pl_.resident) {
      o << ind << "#pragma unroll\n" << ind << "for (int it = 0; it < " << pl_.iters << "; ++it) {\n";
      o << ind << "  const long q = (long)it * " << pl_.L << " + lane;\n";
      const bool guard_q = pl_.qn % pl_.L != 0;
      o << ind << "  if (" << (guard_q ? "q < " + qn : std::string("true")) << (guard_live ? " && live" : "") << ") {\n";
    } else {
      std::string start = split_parts ? "(long)part * " + std::to_string(pl_.L) + " + lane" : "(long)lane";
      std::string step = std::to_string((long)pl_.L * (split_parts ? pl_.P : 1)) + "L";
      // Four steps unrolled: four loads of each value in flight per lane.
      o << ind << "#pragma unroll 4\n";
      o << ind << "for (long q = " << start << "; q < " << (guard_live ? "(live ? " + qn + " : 0L)" : qn)
        << "; q += " << step << ") {\n";
      o << ind << "  {\n";
    }
    std::string in = ind + "    ";
    o << in << "const long pos = q * " << pl_.W << "L;\n";
    delinearize(in, "pos", pl_.swept);
    body(in);
    o << ind << "  }\n" << ind << "}\n";
  }

  void delinearize(const std::string& ind, const std::string& lin, const std::vector<int>& axes) {
    if (axes.empty()) return;
    o_ << ind << "{\n" << ind << "  long r = " << lin << ";\n";
    for (size_t j = 0; j < axes.size(); ++j) {
      int k = axes[j];
      if (j + 1 == axes.size()) {
        o_ << ind << "  i" << k << " = r;\n";
      } else {
        o_ << ind << "  i" << k << " = r % " << pl_.E[k] << "L; r /= " << pl_.E[k] << "L;\n";
      }
    }
    o_ << ind << "}\n";
  }

  // The identity state of a fold, component j.
  static std::string identity(int kind, int j) {
    switch (kind) {
      case TH_FOLD_SUM: return "0.0f";
      case TH_FOLD_PROD: return "1.0f";
      case TH_FOLD_MAX: return "(-__builtin_inff())";
      case TH_FOLD_MIN: return "__builtin_inff()";
      case TH_FOLD_EXP: return j == 0 ? "(-__builtin_inff())" : "0.0f";
      case TH_FOLD_LINEAR: return j == 0 ? "1.0f" : "0.0f";
      case TH_FOLD_ARGMAX: return j == 0 ? "(-__builtin_inff())" : "__builtin_inff()";
      case TH_FOLD_ARGMIN: return "__builtin_inff()";
      default: return "0.0f";
    }
  }

  // a <- combine(a, b), for component names a[j], b[j].
  static std::string combine(int kind, const std::vector<std::string>& a, const std::vector<std::string>& b) {
    switch (kind) {
      case TH_FOLD_SUM: return a[0] + " = " + a[0] + " + " + b[0] + ";";
      case TH_FOLD_PROD: return a[0] + " = " + a[0] + " * " + b[0] + ";";
      case TH_FOLD_MAX: return a[0] + " = fmaxf(" + a[0] + ", " + b[0] + ");";
      case TH_FOLD_MIN: return a[0] + " = fminf(" + a[0] + ", " + b[0] + ");";
      case TH_FOLD_EXP: return "th_exp_comb(" + a[0] + ", " + a[1] + ", " + b[0] + ", " + b[1] + ");";
      case TH_FOLD_LINEAR: return "th_lin_comb(" + a[0] + ", " + a[1] + ", " + b[0] + ", " + b[1] + ");";
      case TH_FOLD_ARGMAX: return "th_amax_comb(" + a[0] + ", " + a[1] + ", " + b[0] + ", " + b[1] + ");";
      case TH_FOLD_ARGMIN: return "th_amin_comb(" + a[0] + ", " + a[1] + ", " + b[0] + ", " + b[1] + ");";
      default: return "th_sq_comb(" + a[0] + ", " + a[1] + ", " + a[2] + ", " + b[0] + ", " + b[1] + ", " + b[2] + ");";
    }
  }

  static std::vector<std::string> comps(const std::string& base, int k) {
    std::vector<std::string> v;
    for (int j = 0; j < k; ++j) v.push_back(base + "_" + std::to_string(j));
    return v;
  }

  // Merge the lanes of an item's part: every lane ends with the merged state.
  void merge_lanes(const std::string& ind, int kind, const std::vector<std::string>& c) {
    std::ostringstream& o = o_;
    const int K = (int)c.size();
    if (pl_.L == 1) return;
    o << ind << "{\n";
    std::string in = ind + "  ";
    if (pl_.S == 1 && pl_.L % 64 == 0) {
      // Within a wave: butterfly, the lower lane's state first, so that both
      // lanes of a pair hold the same merged state.
      o << in << "const int w = threadIdx.x & 63;\n";
      o << in << "#pragma unroll\n" << in << "for (int o = 32; o > 0; o >>= 1) {\n";
      std::vector<std::string> av, bv;
      for (int j = 0; j < K; ++j) {
        o << in << "  const float p" << j << " = __shfl_xor(" << c[j] << ", o, 64);\n";
        o << in << "  float a" << j << " = (w & o) ? p" << j << " : " << c[j] << ";\n";
        o << in << "  float b" << j << " = (w & o) ? " << c[j] << " : p" << j << ";\n";
        av.push_back("a" + std::to_string(j));
        bv.push_back("b" + std::to_string(j));
      }
      o << in << "  " << combine(kind, av, bv) << "\n";
      for (int j = 0; j < K; ++j) o << in << "  " << c[j] << " = a" << j << ";\n";
      o << in << "}\n";
      const int waves = pl_.L / 64;
      if (waves > 1) {
        for (int j = 0; j < K; ++j)
          o << in << "if (w == 0) th_lds[(threadIdx.x >> 6) * " << K << " + " << j << "] = " << c[j] << ";\n";
        o << in << "__syncthreads();\n";
        std::vector<std::string> bv2;
        for (int j = 0; j < K; ++j) {
          o << in << c[j] << " = th_lds[" << j << "];\n";
          bv2.push_back("b" + std::to_string(j));
        }
        o << in << "for (int u = 1; u < " << waves << "; ++u) {\n";
        for (int j = 0; j < K; ++j) o << in << "  float b" << j << " = th_lds[u * " << K << " + " << j << "];\n";
        o << in << "  " << combine(kind, c, bv2) << "\n" << in << "}\n";
        o << in << "__syncthreads();\n";
      }
    } else {
      // Through LDS, halving (merge_lanes, ext/CUDAExt.jl:997-1014).
      auto at = [&](const std::string& l, int j) {
        return "th_lds[((" + l + ") * " + std::to_string(pl_.S) + " + sidx) * " + std::to_string(K) + " + " +
               std::to_string(j) + "]";
      };
      for (int j = 0; j < K; ++j) o << in << at("lane", j) << " = " << c[j] << ";\n";
      o << in << "for (int h = " << pl_.L / 2 << "; h > 0; h >>= 1) {\n";
      o << in << "  __syncthreads();\n";
      o << in << "  if (lane < h) {\n";
      std::vector<std::string> av, bv;
      for (int j = 0; j < K; ++j) {
        o << in << "    float a" << j << " = " << at("lane", j) << ", b" << j << " = " << at("lane + h", j) << ";\n";
        av.push_back("a" + std::to_string(j));
        bv.push_back("b" + std::to_string(j));
      }
      o << in << "    " << combine(kind, av, bv) << "\n";
      for (int j = 0; j < K; ++j) o << in << "    " << at("lane", j) << " = a" << j << ";\n";
      o << in << "  }\n" << in << "}\n";
      o << in << "__syncthreads();\n";
      for (int j = 0; j < K; ++j) o << in << c[j] << " = " << at("0", j) << ";\n";
      o << in << "__syncthreads();\n";
    }
    o << ind << "}\n";
  }

  // Assign the statistics fold f's merged state gives (to `prefix` + name + `suffix`).
  void observe(const std::string& ind, int f, const std::vector<std::string>& c) { observe_to(ind, f, c, "", ""); }
  // What observation `obs` of a fold of `kind` reads of its state components c.
  static std::string observe_expr(int kind, int obs, const std::vector<std::string>& c) {
    if (kind == TH_FOLD_EXP)
      return obs == TH_OBSERVE_STATISTIC ? c[0] : obs == TH_OBSERVE_SUM ? c[1] : "th_shift(" + c[0] + ") + logf(" + c[1] + ")";
    if (kind == TH_FOLD_SQUARE)
      return obs == TH_OBSERVE_STATISTIC ? "(" + c[0] + " > 0.0f ? " + c[1] + " : __builtin_nanf(\"\"))" : c[2];
    if (kind == TH_FOLD_LINEAR) return obs == TH_OBSERVE_STATISTIC ? c[0] : c[1];
    if (kind == TH_FOLD_ARGMAX || kind == TH_FOLD_ARGMIN) return obs == TH_OBSERVE_STATISTIC ? c[1] : c[0];
    return c[0];
  }

  // One element (y, weight g) into the state components c of a fold of `kind`.
  static std::string step_stmt(int kind, const std::vector<std::string>& c, const std::string& y,
                               const std::string& g) {
    switch (kind) {
      case TH_FOLD_SUM: return c[0] + " += " + y + ";";
      case TH_FOLD_PROD: return c[0] + " *= " + y + ";";
      case TH_FOLD_MAX: return c[0] + " = th_max(" + c[0] + ", " + y + ");";
      case TH_FOLD_MIN: return c[0] + " = th_min(" + c[0] + ", " + y + ");";
      case TH_FOLD_EXP: return "th_exp_step(" + c[0] + ", " + c[1] + ", " + y + ", " + g + ");";
      case TH_FOLD_LINEAR: return "th_lin_step(" + c[0] + ", " + c[1] + ", " + y + ", " + g + ");";
      case TH_FOLD_ARGMAX: return "th_amax_comb(" + c[0] + ", " + c[1] + ", " + y + ", " + g + ");";
      case TH_FOLD_ARGMIN: return "th_amin_comb(" + c[0] + ", " + c[1] + ", " + y + ", " + g + ");";
      default: return "th_sq_step(" + c[0] + ", " + c[1] + ", " + c[2] + ", " + y + ");";
    }
  }

  void observe_to(const std::string& ind, int f, const std::vector<std::string>& c, const std::string& prefix,
                  const std::string& suffix) {
    const int kind = d_->folds[f].kind;
    for (int obs = 0; obs <= TH_OBSERVE_LOGSUMEXP; ++obs) {
      if (!observe_ok(kind, obs)) continue;
      o_ << ind << prefix << stat_name(f, obs) << suffix << " = " << observe_expr(kind, obs, c) << ";\n";
    }
  }

  std::string ws(int f) const { return "w" + std::to_string(f); }

  // Fold the folds of phase index j over this thread's positions, merge the
  // lanes, then observe (one kernel) or keep the part's state (split).
  void fold_phase(const std::string& ind, int j, bool split) {
    std::ostringstream& o = o_;
    const int phase = pl_.phases[j];
    std::vector<int> fs, roots;
    for (int f = 0; f < d_->n_folds; ++f)
      if (d_->folds[f].phase == phase) {
        fs.push_back(f);
        roots.push_back(d_->folds[f].body);
        if (d_->folds[f].weight >= 0) roots.push_back(d_->folds[f].weight);
      }
    o << ind << "{  // phase " << phase << "\n";
    std::string in = ind + "  ";
    std::vector<char> r = reach(d_, roots);
    std::map<int, std::string> hoisted;
    split_emit(in, r, hoisted);
    const std::string vt = pl_.W > 1 ? "th_v" : "float";
    for (int f : fs) {
      const int kind = d_->folds[f].kind;
      for (int c = 0; c < state_size(kind); ++c)
        o << in << vt << " s" << f << "_" << c << " = th_splat(" << identity(kind, c) << ");\n";
    }
    sweep(in, split, [&](const std::string& b) {
      std::map<int, std::string> names;
      std::vector<char> sw(d_->n_terms, 0);
      for (int t = 0; t < d_->n_terms; ++t) sw[t] = r[t] && pl_.dep[t];
      emit(b, sw, pl_.W > 1, pl_.resident, names, &hoisted);
      for (int f : fs) {
        const th_fold& x = d_->folds[f];
        std::string y = name_of(x.body, names, hoisted, pl_.W > 1);
        std::string s = "s" + std::to_string(f);
        switch (x.kind) {
          case TH_FOLD_SUM: o << b << s << "_0 += " << y << ";\n"; break;
          case TH_FOLD_PROD: o << b << s << "_0 *= " << y << ";\n"; break;
          case TH_FOLD_MAX: o << b << s << "_0 = th_max(" << s << "_0, " << y << ");\n"; break;
          case TH_FOLD_MIN: o << b << s << "_0 = th_min(" << s << "_0, " << y << ");\n"; break;
          case TH_FOLD_EXP: {
            std::string g = x.weight >= 0 ? name_of(x.weight, names, hoisted, pl_.W > 1)
                                          : (pl_.W > 1 ? "th_splat(1.0f)" : "1.0f");
            o << b << "th_exp_step(" << s << "_0, " << s << "_1, " << y << ", " << g << ");\n";
            break;
          }
          case TH_FOLD_LINEAR:
            o << b << "th_lin_step(" << s << "_0, " << s << "_1, " << y << ", "
              << name_of(x.weight, names, hoisted, pl_.W > 1) << ");\n";
            break;
          case TH_FOLD_ARGMAX:
          case TH_FOLD_ARGMIN:
            o << b << (x.kind == TH_FOLD_ARGMAX ? "th_amax_comb(" : "th_amin_comb(") << s << "_0, " << s << "_1, "
              << y << ", " << name_of(x.weight, names, hoisted, pl_.W > 1) << ");\n";
            break;
          default:
            o << b << "th_sq_step(" << s << "_0, " << s << "_1, " << s << "_2, " << y << ");\n";
        }
      }
    });
    for (int f : fs) {
      const int kind = d_->folds[f].kind, K = state_size(kind);
      std::vector<std::string> c = comps("m" + std::to_string(f), K);
      // The W components of the thread's state, in order.
      for (int k = 0; k < K; ++k)
        o << in << "float " << c[k] << " = s" << f << "_" << k << (pl_.W > 1 ? "[0]" : "") << ";\n";
      for (int w = 1; w < pl_.W; ++w) {
        std::vector<std::string> b;
        for (int k = 0; k < K; ++k) b.push_back("s" + std::to_string(f) + "_" + std::to_string(k) + "[" + std::to_string(w) + "]");
        o << in << combine(kind, c, b) << "\n";
      }
      merge_lanes(in, kind, c);
      if (split) {
        o << in << "if (lane == 0" << (pl_.items % pl_.S ? " && live" : "") << ") {\n";
        for (int k = 0; k < K; ++k)
          o << in << "  " << ws(f) << "[(item * " << pl_.P << "L + part) * " << K << " + " << k << "] = " << c[k] << ";\n";
        o << in << "}\n";
      } else {
        observe(in, f, c);
      }
    }
    o << ind << "}\n";
  }

  // Merge every part's state of fold f from its workspace, then observe.
  void merge_parts(const std::string& ind, int f) {
    std::ostringstream& o = o_;
    const int kind = d_->folds[f].kind, K = state_size(kind);
    o << ind << "{\n";
    std::string in = ind + "  ";
    std::vector<std::string> c = comps("m" + std::to_string(f), K), b;
    for (int k = 0; k < K; ++k) o << in << "float " << c[k] << " = " << identity(kind, k) << ";\n";
    o << in << "if (" << (pl_.items % pl_.S ? "live" : "true") << ") {\n";
    o << in << "  for (int j = lane; j < " << pl_.P << "; j += " << pl_.L << ") {\n";
    for (int k = 0; k < K; ++k) {
      o << in << "    const float b" << k << " = " << ws(f) << "[(item * " << pl_.P << "L + j) * " << K << " + " << k << "];\n";
      b.push_back("b" + std::to_string(k));
    }
    o << in << "    " << combine(kind, c, b) << "\n" << in << "  }\n" << in << "}\n";
    merge_lanes(in, kind, c);
    observe(in, f, c);
    o << ind << "}\n";
  }

  void store(const std::string& ind, const th_output& x, const std::string& val, bool vec) {
    std::string p = vname(x.value), at = addr(x.index, x.value);
    if (x.accumulate) {  // a fold by key: positions may repeat
      o_ << ind << (pl_.ordered ? "th_add_ordered(" : "th_add(") << p << ", " << at << ", " << val << ");\n";
      return;
    }
    // Full outputs are written once and not read again here: non-temporal.
    const std::string n = x.full ? "n" : "";
    if (!vec || pl_.W == 1) {
      o_ << ind << "th_st" << n << "(" << p << ", " << at << ", " << val << ");\n";
      return;
    }
    const int64_t cv = x.index.coeff[pl_.vax];
    if (cv == 0) {
      o_ << ind << "th_st(" << p << ", " << at << ", (" << val << ")[" << pl_.W - 1 << "]);\n";
    } else if (vector_access(pl_, x.value, x.index)) {
      o_ << ind << "th_st4" << n << "(" << p << ", " << at << ", " << val << ");\n";
    } else {
      o_ << ind << "th_sts4(" << p << ", " << at << ", " << cv << "L, " << val << ");\n";
    }
  }

  void reduction(const std::string& name, int split_phase) {
    std::ostringstream& o = o_;
    const bool split = pl_.P > 1;
    header(name);
    const int K3 = 3;
    const int lds = std::max(pl_.S * pl_.L, pl_.L / 64 + 1) * K3;
    o << "  __shared__ float th_lds[" << lds << "];\n  (void)th_lds;\n";
    for (int f = 0; f < d_->n_folds; ++f)
      o << "  float* " << ws(f) << " = (float*)a.p[" << d_->n_values + f << "]; (void)" << ws(f) << ";\n";
    if (pl_.S == 1) {
      o << "  const int lane = threadIdx.x, sidx = 0;\n";
    } else {
      o << "  const int lane = threadIdx.x / " << pl_.S << ", sidx = threadIdx.x % " << pl_.S << ";\n";
    }
    o << "  (void)sidx;\n";
    if (pl_.P == 1) {
      o << "  const long blk = blockIdx.x; const int part = 0;\n";
    } else {
      o << "  const long blk = blockIdx.x / " << pl_.P << "; const int part = blockIdx.x % " << pl_.P << ";\n";
    }
    o << "  (void)part;\n";
    o << "  const long item = blk * " << pl_.S << "L + sidx;\n";
    o << "  const bool live = item < " << pl_.items << "L;\n  (void)live;\n";
    // A thread past the last item takes item 0's positions: terms hoisted out
    // of the sweep are evaluated by every thread, and must stay in bounds.
    delinearize("  ", pl_.items % pl_.S ? "(live ? item : 0L)" : "item", pl_.kept);
    for (int f = 0; f < d_->n_folds; ++f)
      for (int obs = 0; obs <= TH_OBSERVE_LOGSUMEXP; ++obs)
        if (observe_ok(d_->folds[f].kind, obs)) o << "  float " << stat_name(f, obs) << " = 0.0f; (void)" << stat_name(f, obs) << ";\n";
    // Registers holding the swept loads, filled once.
    if (pl_.resident) {
      for (int t = 0; t < d_->n_terms; ++t)
        if (d_->terms[t].op == TH_TERM_LOAD && pl_.dep[t])
          o << "  th_v c" << t << "[" << pl_.iters << "];\n";
      o << "  #pragma unroll\n  for (int it = 0; it < " << pl_.iters << "; ++it) {\n";
      o << "    const long q = (long)it * " << pl_.L << " + lane;\n";
      o << "    if (q < " << pl_.qn << "L" << (pl_.items % pl_.S ? " && live" : "") << ") {\n";
      o << "      const long pos = q * " << pl_.W << "L;\n";
      delinearize("      ", "pos", pl_.swept);
      std::map<int, std::string> none;
      for (int t = 0; t < d_->n_terms; ++t)
        if (d_->terms[t].op == TH_TERM_LOAD && pl_.dep[t])
          o << "      c" << t << "[it] = " << term_expr(t, pl_.W > 1, false, none, true) << ";\n";
      o << "    } else {\n";
      for (int t = 0; t < d_->n_terms; ++t)
        if (d_->terms[t].op == TH_TERM_LOAD && pl_.dep[t]) o << "      c" << t << "[it] = th_splat(0.0f);\n";
      o << "    }\n  }\n";
    }
    if (!split) {
      for (size_t j = 0; j < pl_.phases.size(); ++j) fold_phase("  ", (int)j, false);
    } else {
      // Earlier phases from their workspaces; this stage's phase, or none.
      const size_t upto = split_phase >= 0 ? (size_t)split_phase : pl_.phases.size();
      for (int f = 0; f < d_->n_folds; ++f) {
        size_t pj = std::find(pl_.phases.begin(), pl_.phases.end(), d_->folds[f].phase) - pl_.phases.begin();
        if (pj < upto) merge_parts("  ", f);
      }
      if (split_phase >= 0) {
        fold_phase("  ", split_phase, true);
        o << "}\n";
        return;
      }
    }
    // Once per item: the folds' results and the statistics' outputs.
    std::vector<int> once, full;
    for (int x = 0; x < d_->n_outputs; ++x) (d_->outputs[x].full ? full : once).push_back(x);
    if (!once.empty()) {
      o << "  if (lane == 0 && part == 0 && live) {\n";
      for (int k : pl_.swept) o << "    i" << k << " = 0;\n";
      std::vector<int> roots;
      for (int x : once) out_roots(roots, x);
      std::map<int, std::string> names;
      emit("    ", reach(d_, roots), false, false, names, nullptr);
      for (int x : once) store("    ", d_->outputs[x], names.at(d_->outputs[x].term), false);
      o << "  }\n";
    }
    if (!full.empty()) {
      std::vector<int> roots;
      for (int x : full) out_roots(roots, x);
      std::vector<char> r = reach(d_, roots);
      o << "  {\n";
      std::map<int, std::string> hoisted;
      split_emit("    ", r, hoisted);
      sweep("    ", split, [&](const std::string& b) {
        std::map<int, std::string> names;
        std::vector<char> sw(d_->n_terms, 0);
        for (int t = 0; t < d_->n_terms; ++t) sw[t] = r[t] && pl_.dep[t];
        emit(b, sw, pl_.W > 1, pl_.resident, names, &hoisted);
        for (int x : full) {
          const th_output& out = d_->outputs[x];
          store(b, out, name_of(out.term, names, hoisted, pl_.W > 1), true);
        }
      });
      o << "  }\n";
    }
    o << "}\n";
  }

  // One thread per item sweeps the scanned positions in order; at each, the
  // folds take their elements in (phase, index) order (an exclusive scan's
  // result read before its element, an inclusive one's after), then the
  // full outputs; the plain folds' results and the once outputs after.
  void scan(const std::string& name) {
    if (pl_.rows) {
      scan_rows(name);
      return;
    }
    std::ostringstream& o = o_;
    header(name);
    o << "  const long item = (long)blockIdx.x * " << pl_.S << " + threadIdx.x;\n";
    o << "  if (item >= " << pl_.items << "L) return;\n";
    delinearize("  ", "item", pl_.kept);
    for (int f = 0; f < d_->n_folds; ++f) {
      for (int obs = 0; obs <= TH_OBSERVE_LOGSUMEXP; ++obs)
        if (observe_ok(d_->folds[f].kind, obs)) o << "  float " << stat_name(f, obs) << " = 0.0f; (void)" << stat_name(f, obs) << ";\n";
      for (int c = 0; c < state_size(d_->folds[f].kind); ++c)
        o << "  float s" << f << "_" << c << " = " << identity(d_->folds[f].kind, c) << ";\n";
    }
    auto comps_of = [&](int f) { return comps("s" + std::to_string(f), state_size(d_->folds[f].kind)); };
    o << "  for (long q = 0; q < " << pl_.count << "L; ++q) {\n";
    o << "    const long pos = " << (pl_.reverse ? std::to_string(pl_.count - 1) + "L - q" : std::string("q")) << ";\n";
    delinearize("    ", "pos", pl_.swept);
    std::map<int, std::string> names;
    for (int f : pl_.order) {
      const th_fold& x = d_->folds[f];
      if (x.scan == TH_SCAN_EXCLUSIVE) observe("    ", f, comps_of(f));
      std::vector<int> roots{x.body};
      if (x.weight >= 0) roots.push_back(x.weight);
      emit("    ", reach(d_, roots), false, false, names, nullptr);
      const std::string y = names.at(x.body), sf = "s" + std::to_string(f);
      switch (x.kind) {
        case TH_FOLD_SUM: o << "    " << sf << "_0 += " << y << ";\n"; break;
        case TH_FOLD_PROD: o << "    " << sf << "_0 *= " << y << ";\n"; break;
        case TH_FOLD_MAX: o << "    " << sf << "_0 = th_max(" << sf << "_0, " << y << ");\n"; break;
        case TH_FOLD_MIN: o << "    " << sf << "_0 = th_min(" << sf << "_0, " << y << ");\n"; break;
        case TH_FOLD_EXP:
          o << "    th_exp_step(" << sf << "_0, " << sf << "_1, " << y << ", "
            << (x.weight >= 0 ? names.at(x.weight) : std::string("1.0f")) << ");\n";
          break;
        case TH_FOLD_LINEAR:
          o << "    th_lin_step(" << sf << "_0, " << sf << "_1, " << y << ", " << names.at(x.weight) << ");\n";
          break;
        case TH_FOLD_ARGMAX:
        case TH_FOLD_ARGMIN:
          o << "    " << (x.kind == TH_FOLD_ARGMAX ? "th_amax_comb(" : "th_amin_comb(") << sf << "_0, " << sf
            << "_1, " << y << ", " << names.at(x.weight) << ");\n";
          break;
        default:
          o << "    th_sq_step(" << sf << "_0, " << sf << "_1, " << sf << "_2, " << y << ");\n";
      }
      if (x.scan == TH_SCAN_INCLUSIVE) observe("    ", f, comps_of(f));
    }
    std::vector<int> full, once;
    for (int x = 0; x < d_->n_outputs; ++x) (d_->outputs[x].full ? full : once).push_back(x);
    std::vector<int> roots;
    for (int x : full) out_roots(roots, x);
    emit("    ", reach(d_, roots), false, false, names, nullptr);
    for (int x : full) store("    ", d_->outputs[x], names.at(d_->outputs[x].term), false);
    o << "  }\n";
    for (int f = 0; f < d_->n_folds; ++f)
      if (d_->folds[f].scan == TH_SCAN_NONE) observe("  ", f, comps_of(f));
    if (!once.empty()) {
      for (int k : pl_.swept) o << "  i" << k << " = 0;\n";
      std::vector<int> r2;
      for (int x : once) out_roots(r2, x);
      std::map<int, std::string> names2;
      emit("  ", reach(d_, r2), false, false, names2, nullptr);
      for (int x : once) store("  ", d_->outputs[x], names2.at(d_->outputs[x].term), false);
    }
    o << "}\n";
  }

  // A's state components as lift(y, g): the element's own state.
  static std::vector<std::string> lift(int kind, const std::string& y, const std::string& g) {
    switch (kind) {
      case TH_FOLD_EXP: return {y, g};
      case TH_FOLD_SQUARE: return {"1.0f", y, "0.0f"};
      case TH_FOLD_LINEAR:
      case TH_FOLD_ARGMAX:
      case TH_FOLD_ARGMIN: return {y, g};
      default: return {y};
    }
  }

  // The scan of one item by its workgroup: chunks of L x W positions in scan
  // order; each lane scans its W positions, the lanes' totals are scanned
  // across the wave by shuffles (the earlier state always first: the linear
  // fold's combine does not commute) and across waves through LDS, and the
  // chunk's total is carried into the next.  At each position a fold's result
  // is what later folds and the full outputs read.
  void scan_rows(const std::string& name) {
    std::ostringstream& o = o_;
    header(name);
    const int W = pl_.W, L = pl_.L, waves = L / 64;
    const std::string vt = W > 1 ? "th_v" : "float";
    o << "  __shared__ float th_lds[" << waves * 3 << "];\n";
    o << "  const int lane = threadIdx.x, wl = threadIdx.x & 63, wave = threadIdx.x >> 6;\n";
    o << "  const long item = blockIdx.x;\n";
    delinearize("  ", "item", pl_.kept);
    for (int f = 0; f < d_->n_folds; ++f) {
      const int kind = d_->folds[f].kind;
      for (int obs = 0; obs <= TH_OBSERVE_LOGSUMEXP; ++obs)
        if (observe_ok(kind, obs)) {
          o << "  float " << stat_name(f, obs) << " = 0.0f; (void)" << stat_name(f, obs) << ";\n";
          o << "  " << vt << " s" << stat_name(f, obs) << "; (void)s" << stat_name(f, obs) << ";\n";
        }
      for (int c = 0; c < state_size(kind); ++c)
        o << "  float c" << f << "_" << c << " = " << identity(kind, c) << ";\n";  // the carry
    }
    const int64_t chunk = (int64_t)L * W;
    o << "  for (long c0 = 0; c0 < " << pl_.count << "L; c0 += " << chunk << "L) {\n";
    o << "    const long p0 = c0 + (long)lane * " << W << ";\n";
    o << "    const bool ok = p0 < " << pl_.count << "L;\n";
    o << "    const long pos = ok ? " << (pl_.reverse ? std::to_string(pl_.count - 1) + "L - p0" : std::string("p0"))
      << " : 0L;\n";
    delinearize("    ", "pos", pl_.swept);
    stat_vec_ = true;
    std::map<int, std::string> names;
    const std::string in = "    ";
    for (int f : pl_.order) {
      const th_fold& x = d_->folds[f];
      const int kind = x.kind, K = state_size(kind);
      std::vector<int> roots{x.body};
      if (x.weight >= 0) roots.push_back(x.weight);
      emit(in, reach(d_, roots), W > 1, false, names, nullptr);
      const std::string y = names.at(x.body);
      const std::string g = x.weight >= 0 ? names.at(x.weight) : (W > 1 ? "th_splat(1.0f)" : "1.0f");
      const std::string F = std::to_string(f);
      // This lane's prefix states over its W positions: l<f>_<j>_<k>.
      for (int j = 0; j < W; ++j) {
        const std::string yj = W > 1 ? "(" + y + ")[" + std::to_string(j) + "]" : y;
        const std::string gj = W > 1 ? "(" + g + ")[" + std::to_string(j) + "]" : g;
        std::vector<std::string> el = lift(kind, yj, gj), cur;
        for (int k = 0; k < K; ++k) {
          const std::string nm = "l" + F + "_" + std::to_string(j) + "_" + std::to_string(k);
          cur.push_back(nm);
          if (j == 0) o << in << "float " << nm << " = ok ? " << el[k] << " : " << identity(kind, k) << ";\n";
          else o << in << "float " << nm << " = l" << F << "_" << j - 1 << "_" << k << ";\n";
        }
        if (j > 0) {
          std::vector<std::string> e2;
          for (int k = 0; k < K; ++k) {
            const std::string en = "e" + F + "_" + std::to_string(j) + "_" + std::to_string(k);
            o << in << "const float " << en << " = " << el[k] << ";\n";
            e2.push_back(en);
          }
          o << in << "if (ok) { " << combine(kind, cur, e2) << " }\n";
        }
      }
      // The lanes' totals scanned: t (inclusive within the wave), then the
      // exclusive prefix of this lane within the chunk, b.
      std::vector<std::string> t = comps("t" + F, K), b = comps("b" + F, K), q = comps("q" + F, K), a = comps("a" + F, K);
      for (int k = 0; k < K; ++k) o << in << "float " << t[k] << " = l" << F << "_" << W - 1 << "_" << k << ";\n";
      o << in << "#pragma unroll\n" << in << "for (int o = 1; o < 64; o <<= 1) {\n";
      for (int k = 0; k < K; ++k) o << in << "  float " << q[k] << " = __shfl_up(" << t[k] << ", o, 64);\n";
      o << in << "  if (wl >= o) { " << combine(kind, q, t) << " ";
      for (int k = 0; k < K; ++k) o << t[k] << " = " << q[k] << "; ";
      o << "}\n" << in << "}\n";
      for (int k = 0; k < K; ++k) o << in << "if (wl == 63) th_lds[wave * " << K << " + " << k << "] = " << t[k] << ";\n";
      for (int k = 0; k < K; ++k)
        o << in << "float " << b[k] << " = __shfl_up(" << t[k] << ", 1, 64);\n"
          << in << "if (wl == 0) " << b[k] << " = " << identity(kind, k) << ";\n";
      o << in << "__syncthreads();\n";
      // a: the carry, then every earlier wave's total, then b.
      for (int k = 0; k < K; ++k) o << in << "float " << a[k] << " = c" << F << "_" << k << ";\n";
      o << in << "for (int u = 0; u < wave; ++u) {\n";
      for (int k = 0; k < K; ++k) o << in << "  const float " << q[k] << " = th_lds[u * " << K << " + " << k << "];\n";
      o << in << "  " << combine(kind, a, q) << "\n" << in << "}\n";
      o << in << combine(kind, a, b) << "\n";
      // The chunk's total into the carry (every lane alike).
      o << in << "for (int u = 0; u < " << waves << "; ++u) {\n";
      for (int k = 0; k < K; ++k) o << in << "  const float " << q[k] << " = th_lds[u * " << K << " + " << k << "];\n";
      std::vector<std::string> cc = comps("c" + F, K);
      o << in << "  " << combine(kind, cc, q) << "\n" << in << "}\n";
      o << in << "__syncthreads();\n";
      if (x.scan != TH_SCAN_NONE) {
        // This lane's results: a then its positions' prefixes (exclusive: the one before).
        for (int j = 0; j < W; ++j) {
          std::vector<std::string> r = comps("r" + F + "_" + std::to_string(j), K), lj;
          for (int k = 0; k < K; ++k) o << in << "float " << r[k] << " = " << a[k] << ";\n";
          const int upto = x.scan == TH_SCAN_INCLUSIVE ? j : j - 1;
          if (upto >= 0) {
            for (int k = 0; k < K; ++k) lj.push_back("l" + F + "_" + std::to_string(upto) + "_" + std::to_string(k));
            o << in << combine(kind, r, lj) << "\n";
          }
          observe_to(in, f, r, "s", W > 1 ? "[" + std::to_string(j) + "]" : "");
        }
      }
    }
    std::vector<int> full, once, roots;
    for (int x = 0; x < d_->n_outputs; ++x) (d_->outputs[x].full ? full : once).push_back(x);
    for (int x : full) out_roots(roots, x);
    emit(in, reach(d_, roots), W > 1, false, names, nullptr);
    o << in << "if (ok) {\n";
    for (int x : full) store(in + "  ", d_->outputs[x], names.at(d_->outputs[x].term), W > 1);
    o << in << "}\n";
    stat_vec_ = false;
    o << "  }\n";
    // The plain folds' results, and the once outputs (lane 0).
    for (int f = 0; f < d_->n_folds; ++f)
      if (d_->folds[f].scan == TH_SCAN_NONE) observe("  ", f, comps("c" + std::to_string(f), state_size(d_->folds[f].kind)));
    if (!once.empty()) {
      o << "  if (lane == 0) {\n";
      for (int k : pl_.swept) o << "    i" << k << " = 0;\n";
      std::vector<int> r2;
      for (int x : once) out_roots(r2, x);
      std::map<int, std::string> names2;
      emit("    ", reach(d_, r2), false, false, names2, nullptr);
      for (int x : once) store("    ", d_->outputs[x], names2.at(d_->outputs[x].term), false);
      o << "  }\n";
    }
    o << "}\n";
  }

  void pointwise(const std::string& name) {
    std::ostringstream& o = o_;
    header(name);
    if (pl_.ordered) {
      o << "  if (blockIdx.x != 0 || threadIdx.x != 0) return;\n";
      o << "  for (long lin = 0; lin < " << pl_.qn << "L; ++lin) {\n";
    } else {
      o << "  const long lin = (long)blockIdx.x * " << pl_.S << " + threadIdx.x;\n";
      o << "  if (lin >= " << pl_.qn << "L) return;\n";
    }
    o << "  {\n    long r = lin;\n";
    for (int k = 0; k < pl_.rank; ++k) {
      int64_t e = k == 0 ? pl_.E[0] / pl_.W : pl_.E[k];
      if (k + 1 == pl_.rank) o << "    i" << k << " = r" << (k == 0 ? " * " + std::to_string(pl_.W) + "L" : "") << ";\n";
      else o << "    i" << k << " = (r % " << e << "L)" << (k == 0 ? " * " + std::to_string(pl_.W) + "L" : "")
             << "; r /= " << e << "L;\n";
    }
    o << "  }\n";
    std::vector<int> roots;
    for (int x = 0; x < d_->n_outputs; ++x) out_roots(roots, x);
    std::map<int, std::string> names;
    emit("  ", reach(d_, roots), pl_.W > 1, false, names, nullptr);
    for (int x = 0; x < d_->n_outputs; ++x) store("  ", d_->outputs[x], names.at(d_->outputs[x].term), true);
    if (pl_.ordered) o << "  }\n";
    o << "}\n";
  }
};

// ---- compile and cache ------------------------------------------------------

uint64_t fnv1a(const std::string& s, uint64_t h = 1469598103934665603ull) {
  for (unsigned char c : s) {
    h ^= c;
    h *= 1099511628211ull;
  }
  return h;
}

const char* kOptions[] = {"--offload-arch=gfx950", "-O3", "-std=c++17",
                          // No packed FP32 instructions: plain float code compiles to scalar VALU.
                          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};

// The store's bound in bytes: TEMPEST_HIP_CACHE_CAPACITY (bytes, or with a
// K, M or G suffix), 512 MiB by default; 0 keeps nothing (nothing is read or
// written).  As JULIA_OBJCACHE_CAPACITY bounds the reference's store
// (src/Compiler/runtime/cache.jl:43-45).
long long cache_capacity() {
  const char* e = std::getenv("TEMPEST_HIP_CACHE_CAPACITY");
  if (!e || !*e) return 512LL << 20;
  char* end = nullptr;
  long long v = std::strtoll(e, &end, 10);
  if (end && (*end == 'K' || *end == 'k')) v <<= 10;
  else if (end && (*end == 'M' || *end == 'm')) v <<= 20;
  else if (end && (*end == 'G' || *end == 'g')) v <<= 30;
  return std::max(0LL, v);
}

// Code objects loaded from the store and compiled, in this process.
int64_t g_loaded = 0, g_compiled = 0;

std::string cache_dir() {
  std::string dir;
  if (const char* e = std::getenv("TEMPEST_HIP_CACHE"); e && *e) dir = e;
  else if (const char* x = std::getenv("XDG_CACHE_HOME"); x && *x) dir = std::string(x) + "/tempest_hip";
  else if (const char* h = std::getenv("HOME"); h && *h) dir = std::string(h) + "/.cache/tempest_hip";
  else dir = "/tmp/tempest_hip-" + std::to_string((long)getuid());
  // mkdir -p
  for (size_t i = 1; i <= dir.size(); ++i)
    if (i == dir.size() || dir[i] == '/') (void)mkdir(dir.substr(0, i).c_str(), 0755);
  return dir;
}

struct Compiled {
  std::string key;
  std::string describe;
  std::vector<Stage> stages;
  std::string source;
  std::vector<char> code;
};

std::mutex g_mutex;

// Remove the entries used least recently (the oldest modification time; a
// load touches its entry) until the store holds at most `capacity` bytes,
// keeping `keep`, the entry just written.
void trim(const std::string& dir, long long capacity, const std::string& keep) {
  struct Entry {
    std::string path;
    long long bytes;
    struct timespec used;
  };
  std::vector<Entry> entries;
  long long total = 0;
  if (DIR* dp = opendir(dir.c_str())) {
    while (struct dirent* de = readdir(dp)) {
      std::string name = de->d_name;
      if (name.rfind("floor-", 0) != 0 || name.size() < 6 || name.substr(name.size() - 6) != ".hsaco") continue;
      std::string path = dir + "/" + name;
      struct stat st;
      if (stat(path.c_str(), &st) != 0) continue;
      entries.push_back({path, (long long)st.st_size, st.st_mtim});
      total += st.st_size;
    }
    closedir(dp);
  }
  if (total <= capacity) return;
  std::sort(entries.begin(), entries.end(), [](const Entry& a, const Entry& b) {
    return a.used.tv_sec != b.used.tv_sec ? a.used.tv_sec < b.used.tv_sec : a.used.tv_nsec < b.used.tv_nsec;
  });
  for (const Entry& e : entries) {
    if (total <= capacity) break;
    if (e.path == keep) continue;
    if (std::remove(e.path.c_str()) == 0) total -= e.bytes;
  }
}

// Code object for `source`: from the store on disk, else hiprtc (then kept
// in the store, which is trimmed to its capacity).
int code_object(const std::string& source, const std::string& key, std::vector<char>& code) {
  const long long capacity = cache_capacity();
  const std::string dir = capacity > 0 ? cache_dir() : std::string();
  std::string path = dir + "/floor-" + key + ".hsaco";
  if (capacity > 0) {
    std::ifstream in(path, std::ios::binary);
    if (in) {
      code.assign(std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>());
      if (!code.empty()) {
        (void)utimensat(AT_FDCWD, path.c_str(), nullptr, 0);  // used now
        ++g_loaded;
        return TH_OK;
      }
    }
  }
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, source.c_str(), ("floor-" + key + ".hip").c_str(), 0, nullptr, nullptr) !=
      HIPRTC_SUCCESS)
    return fail(TH_E_COMPILE, "hiprtcCreateProgram failed");
  hiprtcResult r = hiprtcCompileProgram(prog, (int)(sizeof kOptions / sizeof kOptions[0]), kOptions);
  if (r != HIPRTC_SUCCESS) {
    size_t n = 0;
    hiprtcGetProgramLogSize(prog, &n);
    std::string log(n, '\0');
    if (n) hiprtcGetProgramLog(prog, &log[0]);
    hiprtcDestroyProgram(&prog);
    return fail(TH_E_COMPILE, std::string("floor kernel failed to compile: ") + hiprtcGetErrorString(r) + "\n" +
                                   log.substr(0, 4000));
  }
  size_t n = 0;
  hiprtcGetCodeSize(prog, &n);
  code.resize(n);
  hiprtcGetCode(prog, code.data());
  hiprtcDestroyProgram(&prog);
  ++g_compiled;
  if (capacity <= 0) return TH_OK;
  // Keep it: written beside, then renamed into place (a lost write only
  // compiles again).
  std::string tmp = path + ".tmp" + std::to_string((long)getpid());
  {
    std::ofstream out(tmp, std::ios::binary);
    out.write(code.data(), (std::streamsize)code.size());
  }
  if (std::rename(tmp.c_str(), path.c_str()) != 0) std::remove(tmp.c_str());
  trim(dir, capacity, path);
  return TH_OK;
}

int generate(const th_floor_desc* d, Plan& pl, Compiled& c) {
  if (int r = plan(d, pl)) return r;
  Writer w(pl);
  // The key: a first pass names the kernels by a placeholder; the text's hash
  // (with the compiler options) names them for good.
  std::vector<Stage> probe;
  std::string text = w.source(probe, "th_floor_K");
  std::string opts;
  for (const char* o : kOptions) opts += std::string(o) + " ";
  char key[17];
  std::snprintf(key, sizeof key, "%016" PRIx64, fnv1a(text + opts));
  c.key = key;
  Writer w2(pl);
  c.source = w2.source(c.stages, "th_floor_" + c.key);
  c.describe = w2.describe();
  return TH_OK;
}

struct Module {
  hipModule_t module = nullptr;
  std::deque<std::string> names;
  std::map<std::string, hipFunction_t> fns;
};

std::unordered_map<std::string, std::unique_ptr<Module>>& modules() {
  static std::unordered_map<std::string, std::unique_ptr<Module>> m;
  return m;
}

}  // namespace floorgen
}  // namespace th

using namespace th;
using namespace th::floorgen;

extern "C" {

int th_floor_source(const th_floor_desc* desc, char* out, size_t capacity, size_t* needed) {
  Plan pl;
  Compiled c;
  if (int r = generate(desc, pl, c)) return r;
  if (needed) *needed = c.source.size() + 1;
  if (out && capacity) std::snprintf(out, capacity, "%s", c.source.c_str());
  return TH_OK;
}

int th_floor_cache_counts(int64_t* loaded, int64_t* compiled) {
  TH_REQUIRE(loaded && compiled, "th_floor_cache_counts: null output");
  std::lock_guard<std::mutex> lock(g_mutex);
  *loaded = g_loaded;
  *compiled = g_compiled;
  return TH_OK;
}

int th_floor_compile(const th_floor_desc* desc) {
  Plan pl;
  Compiled c;
  if (int r = generate(desc, pl, c)) return r;
  std::lock_guard<std::mutex> lock(g_mutex);
  return code_object(c.source, c.key, c.code);
}

int th_build_floor(const th_floor_desc* desc, th_launch** out) {
  if (int r = require_ready()) return r;
  TH_REQUIRE(out != nullptr, "th_build_floor: null output");
  *out = nullptr;
  Plan pl;
  Compiled c;
  if (int r = generate(desc, pl, c)) return r;
  Module* mod = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_mutex);
    auto it = modules().find(c.key);
    if (it == modules().end()) {
      if (int r = code_object(c.source, c.key, c.code)) return r;
      auto m = std::make_unique<Module>();
      hipError_t e = hipModuleLoadData(&m->module, c.code.data());
      if (e != hipSuccess) {
        // A damaged cache file: compile afresh once.
        if (cache_capacity() > 0) std::remove((cache_dir() + "/floor-" + c.key + ".hsaco").c_str());
        if (int r = code_object(c.source, c.key, c.code)) return r;
        TH_HIP(hipModuleLoadData(&m->module, c.code.data()));
      }
      for (const Stage& s : c.stages) {
        hipFunction_t f;
        TH_HIP(hipModuleGetFunction(&f, m->module, s.name.c_str()));
        m->names.push_back(s.name);
        m->fns[s.name] = f;
      }
      it = modules().emplace(c.key, std::move(m)).first;
    }
    mod = it->second.get();
  }
  const th_floor_desc* d = desc;
  const int nws = pl.reduction && !pl.scan && pl.P > 1 ? d->n_folds : 0;
  struct Args {
    void* p[kMaxArgs];
  } args{};
  for (int v = 0; v < d->n_values; ++v) args.p[v] = d->values[v].ptr;
  Builder b("floor", d->n_values);
  for (int v = 0; v < d->n_values; ++v)
    if (pl.W > 1 && pl.vec_ok[v]) b.align(v, d->values[v].dtype == TH_F32 ? 16 : 8);
  // Workspace: a split fold's partial states, one piece a fold.
  std::vector<uint64_t> at_fold(nws);
  for (int f = 0; f < nws; ++f)
    at_fold[f] = b.workspace((uint64_t)std::max<int64_t>(pl.items, 1) * pl.P * state_size(d->folds[f].kind) *
                             sizeof(float));
  const size_t arg_bytes = sizeof(void*) * (d->n_values + (pl.reduction ? d->n_folds : 0));
  if (pl.items > 0) {
    const int64_t blocks = pl.ordered ? 1 : pl.reduction ? (pl.items + pl.S - 1) / pl.S * pl.P : (pl.qn + pl.S - 1) / pl.S;
    TH_REQUIRE(blocks < (int64_t)1 << 31, "th_build_floor: domain too large for one grid");
    for (const Stage& s : c.stages) {
      int k = b.module_kernel(mod->fns.at(s.name), mod->names[&s - &c.stages[0]].c_str(), dim3((unsigned)blocks),
                              dim3(pl.S * pl.L), 0, args, arg_bytes);
      for (int v = 0; v < d->n_values; ++v) b.ref(v, k, sizeof(void*) * v);
      for (int f = 0; f < nws; ++f) b.ws_ref(k, sizeof(void*) * (d->n_values + f), at_fold[f]);
    }
  }
  // Algorithmic bytes: every value read once, every output written once.
  double bytes = 0;
  for (int v = 0; v < d->n_values; ++v)
    if (pl.read[v]) bytes += (double)d->values[v].length * esize(d->values[v].dtype);
  for (int x = 0; x < d->n_outputs; ++x) {
    const th_floor_value& v = d->values[d->outputs[x].value];
    double n = d->outputs[x].full ? (double)pl.items * (pl.reduction ? pl.count : 1) : (double)pl.items;
    bytes += n * esize(v.dtype);
  }
  b.work(bytes, 0.0, pl.reduction ? (pl.items + pl.S - 1) / pl.S * pl.P : (pl.qn + pl.S - 1) / pl.S);
  *out = b.release();
  (*out)->name = "floor: " + c.describe;
  return TH_OK;
}

}  // extern "C"
