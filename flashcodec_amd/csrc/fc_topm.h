// Top-M selection of PNG-mode deltas, identical to the reference's CPU topk.
//
// png_filter keeps, per (block, feature), the m steps with the largest
// |delta| (flashcodec/codecs/png.py:54-58).  On the CPU torch selects them
// with the C++ standard library's nth_element over (value, index) pairs and
// a value-only comparator ("NaN largest, then >"), so when several |delta|
// tie at the cut the survivors are whichever ones introselect leaves in
// front.  Which tied step survives changes the stored bits, so this file
// restates that selection step by step:
//   introselect: while more than 3 elements remain, pick the median of
//   (first+1, middle, last-1) as pivot, Hoare-partition the rest around it
//   and keep the side holding position m-1; after 2*floor(log2 n) rounds
//   fall back to a heap selection; finish with an insertion sort.
// Ordering keys are the |delta| bit patterns with every NaN mapped to one
// key above +inf, so unsigned comparison equals the reference comparator.
//
// The routine is compiled for the host as well (FC_HD), which is how the
// tests check it against the C++ standard library on the CPU.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define FC_HD __host__ __device__ __forceinline__
#else
#define FC_HD inline
#endif

namespace fc {

struct topm_item {
  uint32_t key;
  uint32_t idx;
};

// Ordering key of a delta: bits of |delta| (sign cleared), NaN -> one key.
FC_HD uint32_t topm_key(uint32_t delta_bits) {
  uint32_t a = delta_bits & 0x7fffffffu;
  return a > 0x7f800000u ? 0x7fc00000u : a;
}

FC_HD bool topm_before(const topm_item& a, const topm_item& b) { return a.key > b.key; }

FC_HD void topm_swap(topm_item* v, int i, int j) {
  topm_item t = v[i];
  v[i] = v[j];
  v[j] = t;
}

FC_HD void topm_sift_up(topm_item* v, int hole, int top, topm_item value) {
  int parent = (hole - 1) / 2;
  while (hole > top && topm_before(v[parent], value)) {
    v[hole] = v[parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  v[hole] = value;
}

// Re-seat `value` into the heap v[0, len) after hole `hole` was vacated.
FC_HD void topm_sift_down(topm_item* v, int hole, int len, topm_item value) {
  const int top = hole;
  int child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (topm_before(v[child], v[child - 1])) child--;
    v[hole] = v[child];
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    v[hole] = v[child - 1];
    hole = child - 1;
  }
  topm_sift_up(v, hole, top, value);
}

// Keep the `mid` best of v[0, len) in v[0, mid).
FC_HD void topm_heap_select(topm_item* v, int mid, int len) {
  if (mid >= 2) {
    for (int parent = (mid - 2) / 2;; --parent) {
      topm_sift_down(v, parent, mid, v[parent]);
      if (parent == 0) break;
    }
  }
  for (int i = mid; i < len; ++i) {
    if (topm_before(v[i], v[0])) {
      topm_item value = v[i];
      v[i] = v[0];
      topm_sift_down(v, 0, mid, value);
    }
  }
}

FC_HD void topm_insertion_sort(topm_item* v, int first, int last) {
  if (first == last) return;
  for (int i = first + 1; i < last; ++i) {
    topm_item val = v[i];
    if (topm_before(val, v[first])) {
      for (int j = i; j > first; --j) v[j] = v[j - 1];
      v[first] = val;
    } else {
      int j = i;
      while (topm_before(val, v[j - 1])) {
        v[j] = v[j - 1];
        --j;
      }
      v[j] = val;
    }
  }
}

// Rearranges v[0, n) so that v[0, m) holds the m selected items.
FC_HD void topm_select(topm_item* v, int n, int m) {
  const int nth = m - 1;
  if (n <= 0 || nth >= n) return;
  int first = 0, last = n;
  int depth = 0;
  for (int t = n; t > 1; t >>= 1) ++depth;
  depth *= 2;
  while (last - first > 3) {
    if (depth == 0) {
      topm_heap_select(v + first, nth + 1 - first, last - first);
      topm_swap(v, first, nth);
      return;
    }
    --depth;
    const int mid = first + (last - first) / 2;
    // median of (first+1, mid, last-1) into `first`
    const int a = first + 1, b = mid, c = last - 1;
    if (topm_before(v[a], v[b])) {
      if (topm_before(v[b], v[c]))
        topm_swap(v, first, b);
      else if (topm_before(v[a], v[c]))
        topm_swap(v, first, c);
      else
        topm_swap(v, first, a);
    } else if (topm_before(v[a], v[c])) {
      topm_swap(v, first, a);
    } else if (topm_before(v[b], v[c])) {
      topm_swap(v, first, c);
    } else {
      topm_swap(v, first, b);
    }
    // Hoare partition of [first+1, last) around v[first]
    int lo = first + 1, hi = last;
    while (true) {
      while (topm_before(v[lo], v[first])) ++lo;
      --hi;
      while (topm_before(v[first], v[hi])) --hi;
      if (!(lo < hi)) break;
      topm_swap(v, lo, hi);
      ++lo;
    }
    if (lo <= nth)
      first = lo;
    else
      last = lo;
  }
  topm_insertion_sort(v, first, last);
}

// Selection mask (bit i set = step i kept) of the m largest of n keys.
// n <= 64, 1 <= m.
FC_HD uint64_t topm_mask_exact(const uint32_t* keys, int n, int m) {
  topm_item v[64];
  for (int i = 0; i < n; ++i) v[i] = topm_item{keys[i], (uint32_t)i};
  topm_select(v, n, m);
  uint64_t mask = 0;
  for (int i = 0; i < m && i < n; ++i) mask |= (uint64_t)1 << v[i].idx;
  return mask;
}

#if defined(__HIPCC__)
// Descending bitonic sort of N (power of two) keys held in registers.
template <int N>
__device__ __forceinline__ void bitonic_sort_desc(uint32_t (&k)[N]) {
#pragma unroll
  for (int size = 2; size <= N; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int j = i ^ stride;
        if (j > i) {
          const bool desc = (i & size) == 0;
          const uint32_t a = k[i], c = k[j];
          const uint32_t hi = a > c ? a : c, lo = a > c ? c : a;
          k[i] = desc ? hi : lo;
          k[j] = desc ? lo : hi;
        }
      }
    }
  }
}

// Keep mask of the `m` largest of `n` keys (n < RMAX).  The common case —
// the m-th and (m+1)-th largest keys differ, or the cut falls on zero,
// where keeping or zeroing a +-0 delta stores the same bits — is decided
// from a sorting network; a nonzero tie across the cut takes the exact
// introselect restatement.
template <int RMAX>
__device__ __forceinline__ uint64_t topm_mask(const uint32_t (&key)[RMAX], int n, int m) {
  uint32_t s[RMAX];
#pragma unroll
  for (int i = 0; i < RMAX; ++i) s[i] = i < n ? key[i] : 0u;
  bitonic_sort_desc<RMAX>(s);
  uint32_t vm = 0, vm1 = 0;
#pragma unroll
  for (int i = 0; i < RMAX; ++i) {
    if (i == m - 1) vm = s[i];
    if (i == m) vm1 = s[i];
  }
  if (vm == 0u || vm != vm1) {
    uint64_t mask = 0;
#pragma unroll
    for (int i = 0; i < RMAX; ++i)
      if (i < n && key[i] >= vm) mask |= (uint64_t)1 << i;
    return mask;
  }
  uint32_t kk[64];
  for (int i = 0; i < n; ++i) kk[i] = key[i];
  return topm_mask_exact(kk, n, m);
}
#endif  // __HIPCC__

}  // namespace fc
