// Minimal static-partition parallel loop over std::thread (the host side
// stays free of a second OpenMP runtime when loaded next to other libraries).
#pragma once

#include <algorithm>
#include <cstddef>
#include <thread>
#include <vector>

namespace l2c_host {

// Calls f(i) for every i in [0, n), split into `threads` contiguous ranges.
template <typename F>
void parallel_for(size_t n, int threads, F f) {
  if (threads <= 1 || n < 4096) {
    for (size_t i = 0; i < n; ++i) f(i);
    return;
  }
  const size_t parts = std::min<size_t>(static_cast<size_t>(threads), n);
  std::vector<std::thread> pool;
  pool.reserve(parts);
  for (size_t p = 0; p < parts; ++p) {
    const size_t begin = n * p / parts, end = n * (p + 1) / parts;
    pool.emplace_back([=] {
      for (size_t i = begin; i < end; ++i) f(i);
    });
  }
  for (auto &t : pool) t.join();
}

// Calls f(begin, end, part) for `parts` contiguous ranges of [0, n).
template <typename F>
void parallel_ranges(size_t n, int threads, F f) {
  const size_t parts = std::max<size_t>(1, std::min<size_t>(static_cast<size_t>(threads), n));
  if (parts == 1) {
    f(size_t(0), n, size_t(0));
    return;
  }
  std::vector<std::thread> pool;
  pool.reserve(parts);
  for (size_t p = 0; p < parts; ++p) {
    const size_t begin = n * p / parts, end = n * (p + 1) / parts;
    pool.emplace_back([=] { f(begin, end, p); });
  }
  for (auto &t : pool) t.join();
}

}  // namespace l2c_host
