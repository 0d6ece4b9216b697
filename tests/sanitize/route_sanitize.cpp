// Drives the host route builder (omniwave_amd/csrc/route.cpp) over a grid of plans, for a build
// with AddressSanitizer and UndefinedBehaviorSanitizer (tests/test_route_sanitizers.py).
//
// Every table is a heap vector of exactly the documented size, so a write or read past it is
// reported.  Checks per plan: the token table holds each of [0, H*W) once and pads (= H*W)
// after; the channel table likewise over [0, C); the space_to_depth output-row table is a
// permutation of the valid rows.  Invalid plans and arguments must fail with an error code.
// Prints "tables <n>" and an FNV-1a digest of the tables of the plans listed on the command
// line ("H W C g d route level"), one line each, so the caller can compare them with the oracle.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "omniwave_amd.h"

namespace {

int g_failures = 0;

void check(bool ok, const char* what, const OwPlan& p) {
  if (ok) return;
  ++g_failures;
  std::fprintf(stderr, "FAIL %s: H=%d W=%d C=%d g=%d d=%d route=%d level=%d window=%d shift=%d\n", what, p.height,
               p.width, p.channels, p.spatial_tile, p.channel_tile, p.route, p.radix_level, p.window, p.shift);
}

bool is_permutation_with_pads(const std::vector<int32_t>& t, int32_t n) {
  std::vector<int> seen(static_cast<size_t>(n), 0);
  for (size_t i = 0; i < t.size(); ++i) {
    const int32_t v = t[i];
    if (i < static_cast<size_t>(n)) {
      if (v < 0 || v >= n || seen[static_cast<size_t>(v)]) return false;
      seen[static_cast<size_t>(v)] = 1;
    } else if (v != n) {
      return false;
    }
  }
  return true;
}

uint64_t fnv(uint64_t h, const std::vector<int32_t>& t) {
  for (int32_t v : t) {
    for (int b = 0; b < 4; ++b) {
      h ^= static_cast<uint8_t>(static_cast<uint32_t>(v) >> (8 * b));
      h *= 1099511628211ull;
    }
  }
  return h;
}

// Builds and checks the tables of one plan; returns their digest (0 if the plan failed).
uint64_t run_plan(const OwPlan& p, bool expect_ok) {
  int32_t q_s = 0, q_c = 0;
  const int rc = ow_plan_dims(&p, &q_s, &q_c);
  if (!expect_ok) {
    check(rc != OW_OK, "invalid plan accepted by ow_plan_dims", p);
    std::vector<int32_t> tok(16), ch(16);
    check(ow_route_build(&p, tok.data(), ch.data()) != OW_OK, "invalid plan accepted by ow_route_build", p);
    return 0;
  }
  check(rc == OW_OK, "ow_plan_dims", p);
  if (rc != OW_OK) return 0;
  const int32_t n = p.height * p.width;
  std::vector<int32_t> tok(static_cast<size_t>(q_s) * p.spatial_tile), ch(static_cast<size_t>(q_c) * p.channel_tile);
  check(ow_route_build(&p, tok.data(), ch.data()) == OW_OK, "ow_route_build", p);
  check(is_permutation_with_pads(tok, n), "token table", p);
  check(is_permutation_with_pads(ch, p.channels), "channel table", p);
  uint64_t h = fnv(fnv(1469598103934665603ull, tok), ch);
  for (int32_t f : {1, 2, 4}) {
    std::vector<int32_t> rows(tok.size());
    const int src = ow_route_s2d_rows(&p, f, tok.data(), rows.data());
    if (p.height % f == 0 && p.width % f == 0) {
      check(src == OW_OK, "ow_route_s2d_rows", p);
      check(is_permutation_with_pads(rows, n), "s2d output rows", p);
      h = fnv(h, rows);
    } else {
      check(src != OW_OK, "indivisible space_to_depth factor accepted", p);
    }
  }
  return h;
}

}  // namespace

int main(int argc, char** argv) {
  const int32_t routes[] = {OW_ROUTE_LOCAL, OW_ROUTE_SHIFTED, OW_ROUTE_RADIX};
  const int32_t hw[] = {1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 13, 14, 16, 28, 56};
  const int32_t chans[] = {1, 5, 64, 96, 128, 200, 512};
  const int32_t gs[] = {1, 3, 16};
  const int32_t ds[] = {1, 16, 64, 128};
  const int32_t wins[][2] = {{4, 2}, {3, 1}, {5, 0}, {2, 3}};
  long n_plans = 0;
  for (int32_t h : hw)
    for (int32_t w : hw)
      for (int32_t route : routes)
        for (const auto& ws : wins) {
          if (route == OW_ROUTE_RADIX && ws[0] != 4) continue;  // window / shift unused by radix
          for (int32_t level = 0; level < (route == OW_ROUTE_RADIX ? 4 : 1); ++level)
            for (int32_t c : chans)
              for (int32_t g : gs)
                for (int32_t d : ds) {
                  if (c > 128 && (h * w) % 7 != 0 && g != 16) continue;  // keep the grid a few seconds long
                  const OwPlan p{h, w, c, g, d, route, level, ws[0], ws[1]};
                  run_plan(p, true);
                  ++n_plans;
                }
        }
  // Invalid plans and arguments.
  const OwPlan bad[] = {{0, 4, 8, 16, 4, OW_ROUTE_LOCAL, 0, 4, 2}, {4, -1, 8, 16, 4, OW_ROUTE_LOCAL, 0, 4, 2},
                        {4, 4, 0, 16, 4, OW_ROUTE_LOCAL, 0, 4, 2}, {4, 4, 8, 0, 4, OW_ROUTE_LOCAL, 0, 4, 2},
                        {4, 4, 8, 16, 0, OW_ROUTE_LOCAL, 0, 4, 2}, {4, 4, 8, 16, 4, 9, 0, 4, 2},
                        {4, 4, 8, 16, 4, OW_ROUTE_RADIX, -1, 4, 2}, {4, 4, 8, 16, 4, OW_ROUTE_LOCAL, 0, 0, 2},
                        {4, 4, 8, 16, 4, OW_ROUTE_SHIFTED, 0, 4, -1}, {65536, 65536, 8, 16, 4, OW_ROUTE_LOCAL, 0, 4, 2}};
  for (const OwPlan& p : bad) run_plan(p, false);
  {
    const OwPlan p{4, 4, 8, 16, 4, OW_ROUTE_LOCAL, 0, 4, 2};
    int32_t q = 0;
    std::vector<int32_t> t(16);
    check(ow_plan_dims(nullptr, &q, &q) != OW_OK, "NULL plan", p);
    check(ow_plan_dims(&p, nullptr, &q) != OW_OK, "NULL q_s", p);
    check(ow_route_build(&p, nullptr, t.data()) != OW_OK, "NULL token table", p);
    check(ow_route_s2d_rows(&p, 0, t.data(), t.data()) != OW_OK, "space_to_depth factor 0", p);
  }
  std::printf("tables %ld\n", n_plans);
  for (int i = 1; i + 6 < argc; i += 7) {
    const OwPlan p{std::atoi(argv[i]), std::atoi(argv[i + 1]), std::atoi(argv[i + 2]), std::atoi(argv[i + 3]),
                   std::atoi(argv[i + 4]), std::atoi(argv[i + 5]), std::atoi(argv[i + 6]), 4, 2};
    int32_t q_s = 0, q_c = 0;
    if (ow_plan_dims(&p, &q_s, &q_c) != OW_OK) return 2;
    std::vector<int32_t> tok(static_cast<size_t>(q_s) * p.spatial_tile), ch(static_cast<size_t>(q_c) * p.channel_tile);
    if (ow_route_build(&p, tok.data(), ch.data()) != OW_OK) return 2;
    std::printf("plan");
    for (int32_t v : tok) std::printf(" %d", v);
    std::printf(" |");
    for (int32_t v : ch) std::printf(" %d", v);
    std::printf("\n");
  }
  if (g_failures) std::fprintf(stderr, "%d failures\n", g_failures);
  return g_failures ? 1 : 0;
}
