// The permutations that the reference's frame sampler gets from std::partial_sort and std::sort
// (src/zonos2-sampler.cpp:40-58). The sampler ranks ids by logit and candidates by probability. Where
// keys are equal, the order comes from the standard library's algorithm, not from the comparator. The
// reference is built against GCC 11's libstdc++, so these functions restate that library's published
// algorithms (bits/stl_algo.h: introsort with median-of-three pivots, depth limit 2*floor(log2 n), a
// 16-element insertion-sort threshold; bits/stl_heap.h: heap select, sift-down then sift-up). Run on
// the same input, they give the same permutation, equal keys included.
//
// Each function works on an array of int ids in place and takes a strict-weak-order predicate
// before(a, b). The loops that libstdc++ leaves unguarded, because a valid order has a sentinel, are
// bounded here as well. With a valid order the bounds never fire. With an invalid one (NaN keys) they
// keep every access inside the array. Callers run these on one thread: on the device they serve the
// rare sampling case where equal keys decide the outcome.
#pragma once

#if defined(__HIPCC__)
#define Z2H_HD __host__ __device__
#else
#define Z2H_HD
#endif

namespace z2h_order {

// Move the hole at `hole` down to a leaf along the children that come first, then put `val` back up
// the path while its parent comes before it. This is libstdc++'s __adjust_heap followed by __push_heap.
template <class Before>
Z2H_HD inline void heap_fix(int * v, int hole, int len, int val, const Before & before) {
    const int top = hole;
    int c = hole;
    while (c < (len - 1) / 2) {
        c = 2 * c + 2;                                    // right child
        if (before(v[c], v[c - 1])) --c;                  // the left one comes first
        v[hole] = v[c];
        hole = c;
    }
    if ((len & 1) == 0 && c == (len - 2) / 2) {           // a last parent with only a left child
        c = 2 * c + 2;
        v[hole] = v[c - 1];
        hole = c - 1;
    }
    for (int up = (hole - 1) / 2; hole > top && before(v[up], val); up = (hole - 1) / 2) {
        v[hole] = v[up];
        hole = up;
    }
    v[hole] = val;
}

// Heap over v[0, len) whose root is the element that comes last in the order.
template <class Before>
Z2H_HD inline void heap_build(int * v, int len, const Before & before) {
    if (len < 2) return;
    for (int p = (len - 2) / 2;; --p) {
        heap_fix(v, p, len, v[p], before);
        if (p == 0) return;
    }
}

// The root leaves to v[slot] and the element held there enters the heap v[0, len).
template <class Before>
Z2H_HD inline void heap_swap_root(int * v, int len, int slot, const Before & before) {
    const int val = v[slot];
    v[slot] = v[0];
    heap_fix(v, 0, len, val, before);
}

// std::partial_sort(v, v + mid, v + n, before): v[0, mid) ends up sorted and holds the mid elements
// that come first. Heap select over the rest, then sort the heap.
template <class Before>
Z2H_HD inline void partial_order(int * v, int mid, int n, const Before & before) {
    heap_build(v, mid, before);
    for (int i = mid; i < n; ++i)
        if (before(v[i], v[0])) heap_swap_root(v, mid, i, before);
    for (int last = mid - 1; last >= 1; --last) heap_swap_root(v, last, last, before);
}

// Shift v[i] left past the elements that it comes before. lo is a bound that a valid order never reaches.
template <class Before>
Z2H_HD inline void insert_left(int * v, int i, int lo, const Before & before) {
    const int val = v[i];
    int j = i - 1;
    while (j >= lo && before(val, v[j])) { v[j + 1] = v[j]; --j; }
    v[j + 1] = val;
}

template <class Before>
Z2H_HD inline void insertion_order(int * v, int first, int last, const Before & before) {
    for (int i = first + 1; i < last; ++i) {
        if (before(v[i], v[first])) {
            const int val = v[i];
            for (int j = i; j > first; --j) v[j] = v[j - 1];
            v[first] = val;
        } else {
            insert_left(v, i, first, before);
        }
    }
}

// Median of v[a], v[b], v[c] swapped into v[res]: the pivot choice of libstdc++'s introsort.
template <class Before>
Z2H_HD inline void median_to(int * v, int res, int a, int b, int c, const Before & before) {
    int m;
    if (before(v[a], v[b])) m = before(v[b], v[c]) ? b : before(v[a], v[c]) ? c : a;
    else m = before(v[a], v[c]) ? a : before(v[b], v[c]) ? c : b;
    const int t = v[res]; v[res] = v[m]; v[m] = t;
}

// Hoare partition of v[first + 1, last) around the pivot at v[first]. Returns the cut.
template <class Before>
Z2H_HD inline int partition_at_first(int * v, int first, int last, const Before & before) {
    const int mid = first + (last - first) / 2;
    median_to(v, first, first + 1, mid, last - 1, before);
    int f = first + 1, l = last;
    while (true) {
        while (f < last - 1 && before(v[f], v[first])) ++f;
        --l;
        while (l > first && before(v[first], v[l])) --l;
        if (!(f < l)) return f;
        const int t = v[f]; v[f] = v[l]; v[l] = t;
        ++f;
    }
}

// std::sort(v, v + n, before). libstdc++ recurses into the right part and loops on the left. The
// parts are disjoint, so an explicit stack processes them with the same result. Each pending part
// took one level of the depth limit, so the stack holds at most 2*floor(log2 n) + 1 < 64 entries.
template <class Before>
Z2H_HD inline void sort_order(int * v, int n, const Before & before) {
    if (n <= 0) return;
    int lg = 0;
    while ((n >> (lg + 1)) != 0) ++lg;
    int st_first[64], st_last[64], st_depth[64], sp = 0;
    st_first[0] = 0; st_last[0] = n; st_depth[0] = 2 * lg; sp = 1;
    while (sp > 0) {
        --sp;
        const int first = st_first[sp];
        int last = st_last[sp], depth = st_depth[sp];
        while (last - first > 16) {
            if (depth == 0) {                             // heap sort of the part
                partial_order(v + first, last - first, last - first, before);
                break;
            }
            --depth;
            const int cut = partition_at_first(v, first, last, before);
            if (sp < 64) { st_first[sp] = cut; st_last[sp] = last; st_depth[sp] = depth; ++sp; }
            last = cut;
        }
    }
    if (n > 16) {
        insertion_order(v, 0, 16, before);
        for (int i = 16; i < n; ++i) insert_left(v, i, 0, before);
    } else {
        insertion_order(v, 0, n, before);
    }
}

}  // namespace z2h_order
