// Host-side route tables (token and channel index maps) of the BiGEMM backend.
//
// Semantics follow omniweave/models/routing.py:40-179.  The local and shifted token orders
// are built from per-axis window lists instead of the reference's 2-D loop + dedup:
//
//   local   (routing.py:57-65)  window k of an axis of length n covers [k*w, min(k*w+w, n));
//   shifted (routing.py:68-90)  window k covers (k*w - shift + i) mod n, i in [0, w), over
//                               the bases range(-shift, n - shift, w); an axis position
//                               is kept only in the first window (and first slot) that
//                               reaches it.
//
// A token (r, c) first occurs in 2-D window (kr, kc) exactly when kr is the first row window
// holding r and kc the first column window holding c, and inside that window it is emitted
// at (first slot of r, first slot of c).  So the first-occurrence 2-D order equals
// "for kr, for kc, for r in rows'(kr), for c in cols'(kc)" over the deduplicated per-axis
// lists, which is what token_order() writes.
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "ow_common.h"

namespace ow {

namespace {
thread_local char g_error[1024] = {0};
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_error[0] = 0; }

const char* last_error() { return g_error; }

namespace {

using AxisWindows = std::vector<std::vector<int32_t>>;

AxisWindows axis_local(int32_t n, int32_t w) {
  AxisWindows out;
  for (int32_t base = 0; base < n; base += w) {
    std::vector<int32_t> win;
    for (int32_t p = base; p < base + w && p < n; ++p) win.push_back(p);
    out.push_back(std::move(win));
  }
  return out;
}

AxisWindows axis_shifted(int32_t n, int32_t w, int32_t shift) {
  AxisWindows out;
  std::vector<char> seen(static_cast<size_t>(n), 0);
  for (int64_t base = -static_cast<int64_t>(shift); base < static_cast<int64_t>(n) - shift; base += w) {
    std::vector<int32_t> win;
    for (int32_t i = 0; i < w; ++i) {
      int64_t p = (base + i) % n;
      if (p < 0) p += n;
      if (!seen[static_cast<size_t>(p)]) {
        seen[static_cast<size_t>(p)] = 1;
        win.push_back(static_cast<int32_t>(p));
      }
    }
    out.push_back(std::move(win));
  }
  return out;
}

std::vector<int32_t> windowed_order(const AxisWindows& rows, const AxisWindows& cols, int32_t width) {
  std::vector<int32_t> order;
  for (const auto& rw : rows)
    for (const auto& cw : cols)
      for (int32_t r : rw)
        for (int32_t c : cw) order.push_back(r * width + c);
  return order;
}

// routing.py:93-104: tokens grouped by the radix digit at `level` (radix = g).
std::vector<int32_t> radix_token_order(int32_t n, int32_t g, int32_t level) {
  std::vector<int32_t> order;
  int64_t stride = 1;
  for (int32_t i = 0; i < level && stride < n; ++i) stride *= g;
  if (stride >= n) {  // only digit 0 exists: identity
    for (int32_t i = 0; i < n; ++i) order.push_back(i);
    return order;
  }
  const int64_t block = stride * g;
  for (int64_t base = 0; base < n; base += block)
    for (int64_t off = 0; off < stride; ++off)
      for (int64_t digit = 0; digit < g; ++digit) {
        const int64_t idx = base + digit * stride + off;
        if (idx < n) order.push_back(static_cast<int32_t>(idx));
      }
  return order;
}

// routing.py:107-121: channel i joins group i mod n_groups; group list rotated by level.
std::vector<int32_t> channel_order(int32_t c, int32_t d, int32_t level) {
  const int32_t n_groups = (c + d - 1) / d;
  std::vector<int32_t> order;
  order.reserve(static_cast<size_t>(c));
  if (level == 0 || n_groups <= 1) {
    for (int32_t i = 0; i < c; ++i) order.push_back(i);
    return order;
  }
  const int32_t rot = level % n_groups;
  for (int32_t k = 0; k < n_groups; ++k) {
    const int32_t grp = (rot + k) % n_groups;
    for (int32_t i = grp; i < c; i += n_groups) order.push_back(i);
  }
  return order;
}

int validate(const OwPlan* p) {
  OW_CHECK_ARG(p != nullptr, "plan is NULL");
  OW_CHECK_ARG(p->height >= 1 && p->width >= 1, "height/width must be >= 1 (got %d x %d)", p->height, p->width);
  OW_CHECK_ARG(static_cast<int64_t>(p->height) * p->width < (int64_t(1) << 30), "H*W too large");
  OW_CHECK_ARG(p->channels >= 1, "channels must be >= 1 (got %d)", p->channels);
  OW_CHECK_ARG(p->spatial_tile >= 1 && p->channel_tile >= 1, "tiles must be >= 1 (g=%d, d=%d)",
               p->spatial_tile, p->channel_tile);
  OW_CHECK_ARG(p->route >= OW_ROUTE_LOCAL && p->route <= OW_ROUTE_RADIX, "unknown route type: %d", p->route);
  OW_CHECK_ARG(p->radix_level >= 0, "radix_level must be >= 0 (got %d)", p->radix_level);
  OW_CHECK_ARG(p->window >= 1 && p->shift >= 0, "window must be >= 1 and shift >= 0");
  return OW_OK;
}

}  // namespace
}  // namespace ow

extern "C" {

int ow_version(void) { return 100; }

const char* ow_last_error(void) { return ow::last_error(); }

int ow_plan_dims(const OwPlan* plan, int32_t* q_s, int32_t* q_c) {
  if (int rc = ow::validate(plan)) return rc;
  OW_CHECK_ARG(q_s && q_c, "output pointers are NULL");
  const int32_t n = plan->height * plan->width;
  *q_s = (n + plan->spatial_tile - 1) / plan->spatial_tile;
  *q_c = (plan->channels + plan->channel_tile - 1) / plan->channel_tile;
  return OW_OK;
}

int ow_route_build(const OwPlan* plan, int32_t* token_index, int32_t* channel_index) {
  if (int rc = ow::validate(plan)) return rc;
  OW_CHECK_ARG(token_index && channel_index, "output pointers are NULL");
  const int32_t h = plan->height, w = plan->width, c = plan->channels;
  const int32_t n = h * w, g = plan->spatial_tile, d = plan->channel_tile;
  std::vector<int32_t> tokens;
  switch (plan->route) {
    case OW_ROUTE_LOCAL:
      tokens = ow::windowed_order(ow::axis_local(h, plan->window), ow::axis_local(w, plan->window), w);
      break;
    case OW_ROUTE_SHIFTED:
      tokens = ow::windowed_order(ow::axis_shifted(h, plan->window, plan->shift),
                                  ow::axis_shifted(w, plan->window, plan->shift), w);
      break;
    default:
      tokens = ow::radix_token_order(n, g, plan->radix_level);
      break;
  }
  if (static_cast<int32_t>(tokens.size()) != n)
    return ow::fail(OW_ERR_INVALID, "route produced %zu tokens for N=%d", tokens.size(), n);
  const int32_t q_s = (n + g - 1) / g;
  for (int32_t i = 0; i < q_s * g; ++i) token_index[i] = i < n ? tokens[static_cast<size_t>(i)] : n;
  const std::vector<int32_t> chans = ow::channel_order(c, d, plan->radix_level);
  const int32_t q_c = (c + d - 1) / d;
  for (int32_t i = 0; i < q_c * d; ++i) channel_index[i] = i < c ? chans[static_cast<size_t>(i)] : c;
  ow::clear_error();
  return OW_OK;
}

int ow_route_s2d_rows(const OwPlan* plan, int32_t factor, const int32_t* token_index, int32_t* out_rows) {
  if (int rc = ow::validate(plan)) return rc;
  OW_CHECK_ARG(token_index && out_rows, "table pointers are NULL");
  const int32_t h = plan->height, w = plan->width, n = h * w, g = plan->spatial_tile;
  OW_CHECK_ARG(factor >= 1 && h % factor == 0 && w % factor == 0,
               "height %d and width %d must be divisible by factor %d", h, w, factor);
  const int32_t q_s = (n + g - 1) / g, wf = w / factor;
  for (int32_t i = 0; i < q_s * g; ++i) {
    const int32_t t = token_index[i];
    if (t < 0 || t >= n) {
      out_rows[i] = n;
      continue;
    }
    const int32_t r = t / w, c = t % w;
    out_rows[i] = ((r / factor) * wf + c / factor) * factor * factor + (r % factor) * factor + c % factor;
  }
  ow::clear_error();
  return OW_OK;
}

}  // extern "C"
