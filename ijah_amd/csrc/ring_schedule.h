// The issue and wait schedule of the grouped GEMM's two LDS rings (chunk_gemm in moe_batch.hip), as plain constexpr
// C++ so that a host program can check it (tests/test_ring_schedule.py simulates the rings against it).
//
// Per wave: A (the rows) DA steps ahead in RA = DA + 1 slots, B (the wave's tiles) DB steps ahead in RB = DB + 1
// slots; OA and OB requests per step. Issue order: prologue A(0) B(0) A(1) B(1) .. A(DA-1) B(DA-1) B(DA) ..
// B(DB-1); step j then issues A(j + DA) and B(j + DB) (while < NS), after the wait for step j's data and a barrier.
// Requests complete in issue order, so waiting until at most n are outstanding completes all but the last n.
#pragma once

namespace ijah {

// How many requests were issued after A(t) and B(t), counted at step t before it issues: the s_waitcnt vmcnt that
// makes both complete.
template <int OA, int OB, int DA, int DB>
constexpr int after_step(int t, int NS) {
  auto mn = [](int x, int y) { return x < y ? x : y; };
  auto mx = [](int x, int y) { return x > y ? x : y; };
  auto sum_ops = [&](int n) { return OA * mn(n, mx(NS - DA, 0)) + OB * mn(n, mx(NS - DB, 0)); };
  const int pa = mn(DA, NS), pb = mn(DB, NS);
  const int prologue = OA * pa + OB * pb;
  const int total = prologue + sum_ops(t);
  int last = 0;  // one past the position of the later of A(t), B(t)
  if (t < DA) {
    last = (OA + OB) * (t + 1);
  } else if (t < DB) {
    last = mx(prologue + sum_ops(t - DA) + OA, (OA + OB) * pa + OB * (t - pa) + OB);
  } else {
    last = mx(prologue + sum_ops(t - DA) + OA, prologue + sum_ops(t - DB) + ((t - DB) + DA < NS ? OA : 0) + OB);
  }
  return total - last;
}
// Steps t with DB <= t and t + DB < NS (both streams still issuing) wait with one compile-time count: A(t) is the
// later request, followed by B(t - DA + DB) and DA - 1 full steps.
template <int DB>
constexpr bool steady_step(int t, int NS) { return t >= DB && t + DB < NS; }
template <int OA, int OB, int DA>
constexpr int kAfterSteady = OB + (DA - 1) * (OA + OB);
static_assert(after_step<2, 1, 2, 5>(5, 1000) == kAfterSteady<2, 1, 2> &&
                  after_step<1, 1, 2, 5>(9, 1000) == kAfterSteady<1, 1, 2> &&
                  after_step<2, 1, 1, 3>(7, 1000) == kAfterSteady<2, 1, 1>,
              "steady-state wait count");
// The count the k loop waits with at step t: the steady count, else after_step capped at 15 (the 4-bit immediate of
// wait_vm15; a larger count waits as for 15, which only waits longer).
template <int OA, int OB, int DA, int DB>
constexpr int step_wait(int t, int NS) {
  const int n = after_step<OA, OB, DA, DB>(t, NS);
  return steady_step<DB>(t, NS) ? kAfterSteady<OA, OB, DA> : (n < 15 ? n : 15);
}

}  // namespace ijah
