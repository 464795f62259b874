"""Sequential model of torch's CPU `topk` for one row — test infrastructure, see __init__.py.

torch's CPU topk (aten/src/ATen/native/TopKImpl.h, `topk_impl_loop`) fills a queue of
(value, index) pairs in index order and, when k * 64 > n (the K=8, E=256 router case), calls
`std::nth_element(q, q + k - 1, q + n, greater)` and then `std::sort(q, q + k - 1, greater)`;
the k returned slots are q[0..k-1]. With libstdc++ (GCC) these are introselect (median-of-three
pivot, unguarded Hoare partition, heap-select once the 2*floor(log2 n) depth budget runs out,
insertion sort for ranges of <= 3) and, for k - 1 <= 16 elements, a plain insertion sort. Equal
values therefore come back in the order this partition history leaves them in — neither a
lower-index nor a higher-index rule (prototype/moe_router/results.md:125-128,
prototype/moe_router/moe_router_kernels.h:279-287).

This module restates that algorithm from its published description so tests can (1) check it
against torch.topk on tie-laden rows and (2) build tie fixtures for the device, whose emulation
is a wave-parallel restatement of the same partition sequence. `greater(a, b)` is `a > b` on
values (NaN never occurs on the router path).
"""
from __future__ import annotations


class _Row:
    def __init__(self, values, gt=None):
        self.v = list(values)
        self.q = list(range(len(self.v)))          # queue of indices, values looked up
        self.gt = gt or (lambda a, b: self.v[a] > self.v[b])
        self.heap_path = False

    # -- helpers on queue positions --------------------------------------------------------
    def c(self, i, j):
        return self.gt(self.q[i], self.q[j])

    def swap(self, i, j):
        self.q[i], self.q[j] = self.q[j], self.q[i]

    def median_to_first(self, r, a, b, c):
        if self.c(a, b):
            if self.c(b, c):
                self.swap(r, b)
            elif self.c(a, c):
                self.swap(r, c)
            else:
                self.swap(r, a)
        elif self.c(a, c):
            self.swap(r, a)
        elif self.c(b, c):
            self.swap(r, c)
        else:
            self.swap(r, b)

    def partition(self, lo, hi, pivot):
        while True:
            while self.c(lo, pivot):
                lo += 1
            hi -= 1
            while self.c(pivot, hi):
                hi -= 1
            if not lo < hi:
                return lo
            self.swap(lo, hi)
            lo += 1

    def insertion_sort(self, lo, hi):
        for i in range(lo + 1, hi):
            item = self.q[i]
            j = i
            while j > lo and self.gt(item, self.q[j - 1]):
                self.q[j] = self.q[j - 1]
                j -= 1
            self.q[j] = item

    # -- heap helpers (libstdc++ __adjust_heap / __push_heap / __pop_heap / __make_heap) ----
    def push_heap(self, base, hole, top, item):
        parent = (hole - 1) // 2
        while hole > top and self.gt(self.q[base + parent], item):
            self.q[base + hole] = self.q[base + parent]
            hole = parent
            parent = (hole - 1) // 2
        self.q[base + hole] = item

    def adjust_heap(self, base, hole, length, item):
        top = hole
        child = hole
        while child < (length - 1) // 2:
            child = 2 * (child + 1)
            if self.gt(self.q[base + child], self.q[base + child - 1]):
                child -= 1
            self.q[base + hole] = self.q[base + child]
            hole = child
        if (length & 1) == 0 and child == (length - 2) // 2:
            child = 2 * (child + 1)
            self.q[base + hole] = self.q[base + child - 1]
            hole = child - 1
        self.push_heap(base, hole, top, item)

    def make_heap(self, lo, hi):
        n = hi - lo
        if n < 2:
            return
        parent = (n - 2) // 2
        while True:
            self.adjust_heap(lo, parent, n, self.q[lo + parent])
            if parent == 0:
                return
            parent -= 1

    def heap_select(self, lo, mid, hi):
        self.make_heap(lo, mid)
        for i in range(mid, hi):
            if self.gt(self.q[i], self.q[lo]):
                item = self.q[i]
                self.q[i] = self.q[lo]
                self.adjust_heap(lo, 0, mid - lo, item)

    def introselect(self, nth, depth, on_median=None):
        lo, hi = 0, len(self.q)
        while hi - lo > 3:
            if depth == 0:
                self.heap_path = True
                self.heap_select(lo, nth + 1, hi)
                self.swap(lo, nth)
                return
            depth -= 1
            mid = lo + (hi - lo) // 2
            if on_median is not None:
                on_median(self.q[lo + 1], self.q[mid], self.q[hi - 1])
            self.median_to_first(lo, lo + 1, mid, hi - 1)
            cut = self.partition(lo + 1, hi, lo)
            if cut <= nth:
                lo = cut
            else:
                hi = cut
        self.insertion_sort(lo, hi)


def torch_cpu_topk(values, k: int, gt=None, on_median=None):
    """(indices, heap_path_taken) of torch.topk(values, k) on one row, k * 64 > len(values)."""
    n = len(values)
    if k < 1 or k > n or k * 64 <= n:
        raise ValueError("model covers 1 <= k <= n with k * 64 > n (the nth_element branch)")
    row = _Row(values, gt)
    row.introselect(k - 1, 2 * (n.bit_length() - 1), on_median)
    row.insertion_sort(0, k - 1)
    return row.q[:k], row.heap_path


def adversarial_row(n: int = 256, k: int = 8, start: float | None = None):
    """Values that drive the introselect into its heap-select branch: every median-of-three
    candidate is frozen, as it is first met, to the next value of an increasing run of negative
    numbers; everything else stays at 0, so it ties with itself and beats every frozen value.
    Each pivot is then near the minimum of its range, the partition cut lands near the right end,
    and the range shrinks by about two per round until the depth budget is spent."""
    vals = [0.0] * n
    state = {"next": -float(n * 4) if start is None else float(start)}

    def freeze(*ids):
        for i in ids:
            if vals[i] == 0.0:
                vals[i] = state["next"]
                state["next"] += 1.0

    torch_cpu_topk(vals, k, gt=lambda a, b: vals[a] > vals[b],
                   on_median=lambda a, b, c: freeze(a, b, c))
    return vals
