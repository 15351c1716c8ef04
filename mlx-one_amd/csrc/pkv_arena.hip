// pkv_arena.hip -- device-side page allocation for the paged cache.
//
// The reference keeps page ownership on the host: BlockPool refcounts, pins
// and seals (src/mlx_one/engine/block_cache.py:121-326), the arena's segment
// staging (engine/arena.py:90-113) and a page table per layer cache
// (arena.py:172-225), with a copy of the mutable tail page for every clone
// (engine/paged.py:83-91).  Here the same ownership lives in device memory so a
// decode step needs no host bookkeeping and can be replayed as a graph:
//
//   state  [0] free pages (the stack's height)  [1] sticky error bits
//          [16, 16 + C)      free stack of page ids (C = capacity)
//          [16 + C, 16 + 2C) reference count per page
//   table  [slots][max_pages] page ids of each sequence slot, -1 past its end
//   lens   [slots]            tokens of each slot
//
// One page id addresses the same page in every layer's pool (all layers of a
// sequence grow together), so one reservation serves a whole model step.
// Pages are shared by reference count (fork); the first append into a shared,
// partly filled tail page copies it first (copy-on-write), which gives the
// reference's clone semantics without copying tails that are never written.
//
// Every kernel runs as one workgroup: its reads and writes of the stack height
// need no atomics, and it sees a consistent state whatever came before it on
// the stream.  Calls on one state must be ordered (one stream).

#include "pkv_device.h"
#include "pkv_launch.h"

namespace pkv {

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ int cdiv(int a, int b) { return (a + b - 1) / b; }

// Inclusive prefix sum over the workgroup; *total receives the sum.
__device__ __forceinline__ int block_scan_incl(int v, int *s_wave, int *total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int incl = wave_scan_incl(v, lane);
  if (lane == 63) s_wave[wave] = incl;
  __syncthreads();
  int before = 0, sum = 0;
  for (int k = 0; k < kWaves; ++k) {
    const int t = s_wave[k];
    before += k < wave ? t : 0;
    sum += t;
  }
  __syncthreads();  // s_wave is reused by the next scan
  *total = sum;
  return incl + before;
}

struct ArenaRefs {
  int32_t *top, *err, *stack, *ref;
  __device__ ArenaRefs(const ArenaArgs &a)
      : top(a.state), err(a.state + 1), stack(a.state + kArenaHeaderWords),
        ref(a.state + kArenaHeaderWords + a.capacity) {}
};

__global__ void arena_init_kernel(int32_t *state, int capacity) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < kArenaHeaderWords) state[i] = i == 0 ? capacity : 0;
  if (i < capacity) {
    state[kArenaHeaderWords + i] = capacity - 1 - (int)i;  // pops hand out 0, 1, 2, ...
    state[kArenaHeaderWords + capacity + i] = 0;
  }
}

// Reserve pages for `count` slots growing by arg[i] tokens each (slots distinct).
// The batch row of slot i gets the slot's page ids (entries past them are not
// written: the kernels read a row only up to its length).  A slot that cannot
// grow (its table is full, or the stack is short -- then no slot of the chunk
// grows) keeps its length, its batch length is 0 and its batch row holds -1
// from the page its first new token would go to, so no append (positioned by
// the start or by the batch length) writes anything.
//
// Order of work, to overlap the dependent memory round trips: lengths and tail
// page ids; the copy of each row's existing entries (in flight while) the
// reference-count checks, the prefix sum of the pages needed and the pops.
__global__ __launch_bounds__(kThreads) void arena_reserve_kernel(ArenaArgs a) {
  __shared__ int s_wave[kWaves];
  __shared__ int s_top, s_fail, s_ncow;
  __shared__ int s_slot[kThreads], s_old[kThreads], s_base[kThreads];
  __shared__ int s_cow_src[kThreads], s_cow_dst[kThreads];
  const ArenaRefs r(a);
  const int P = a.page_tokens, mp = a.max_pages;
  if (threadIdx.x == 0) s_top = *r.top;  // only this kernel moves it while it runs
  for (int c0 = 0; c0 < a.count; c0 += kThreads) {
    const int i = c0 + threadIdx.x;
    int s = -1, w = 0, L = 0, nl = 0, oldp = 0, need = 0, tail = -1;
    bool cow = false, blocked = false;
    if (i < a.count) {
      s = a.slots[i];
      w = a.arg[i];
      if (s < 0 || s >= a.num_slots || w < 0) {
        atomicOr(r.err, kArenaBadArgument);
        s = -1;
      } else {
        L = a.lens[s];
        nl = L + w;
        oldp = cdiv(L, P);
        if ((int64_t)nl > (int64_t)mp * P) {
          atomicOr(r.err, kArenaTableFull);
          blocked = true;
        } else if (w > 0 && L % P != 0) {
          tail = a.table[(int64_t)s * mp + L / P];
          if (tail < 0 || tail >= a.capacity) {
            atomicOr(r.err, kArenaCorrupt);
            blocked = true;
          }
        }
      }
    }
    s_slot[threadIdx.x] = s;
    s_old[threadIdx.x] = s >= 0 ? oldp : 0;
    // the rows' existing entries: flattened copy, four entries per item when
    // rows are 16-byte aligned (max_pages % 4 == 0); its loads stay in flight
    // through the reference-count checks below
    const int rows = min(kThreads, a.count - c0);
    {
      const int V = mp % 4 == 0 ? 4 : 1;  // entries per item
      const int items = s >= 0 ? cdiv(oldp, V) : 0;
      int total_items;
      const int incl_items = block_scan_incl(items, s_wave, &total_items);
      s_base[threadIdx.x] = incl_items - items;
      __syncthreads();
      for (int e0 = threadIdx.x; e0 < total_items; e0 += 4 * kThreads) {
        u4 val[4];
        int64_t dst[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int e = e0 + u * kThreads;
          dst[u] = -1;
          if (e < total_items) {
            int lo = 0, hi = rows - 1;  // the last row whose base <= e
            while (lo < hi) {
              const int mid = (lo + hi + 1) >> 1;
              if (s_base[mid] <= e) lo = mid; else hi = mid - 1;
            }
            const int p = (e - s_base[lo]) * V;
            dst[u] = (int64_t)(c0 + lo) * mp + p;
            const int32_t *src = a.table + (int64_t)s_slot[lo] * mp + p;
            if (V == 4) val[u] = *(const u4 *)src;
            else val[u].x = *src;
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (dst[u] < 0) continue;
          if (V == 4) *(u4 *)(a.batch_table + dst[u]) = val[u];
          else a.batch_table[dst[u]] = (int)val[u].x;
        }
      }
    }
    // copy-on-write decisions: a tail held by this slot alone is written in place
    if (tail >= 0 && !blocked) {
      if (r.ref[tail] > 1) {
        if (atomicSub(&r.ref[tail], 1) > 1) cow = true;  // still shared: write into a copy
        else atomicAdd(&r.ref[tail], 1);                 // the others let go meanwhile
      }
    }
    if (blocked) nl = L;
    const int newp = cdiv(nl, P);
    need = s >= 0 ? newp - oldp + (cow ? 1 : 0) : 0;
    int total;
    const int incl = block_scan_incl(need, s_wave, &total);
    if (threadIdx.x == 0) {
      s_fail = s_top < total;
      if (s_fail) atomicOr(r.err, kArenaOutOfPages);
      s_ncow = 0;
    }
    __syncthreads();
    const int top = s_top;
    if (s >= 0 && s_fail && w > 0) {
      if (cow) atomicAdd(&r.ref[tail], 1);  // nothing taken: give the reference back
      blocked = true;
      nl = L;
    }
    int64_t brow = (int64_t)i * mp;
    if (s >= 0 && !s_fail && !blocked) {
      int pos = top - 1 - (incl - need);  // this slot's pages: stack[pos], stack[pos - 1], ...
      if (cow) {
        const int np = r.stack[pos--];
        if (np >= 0 && np < a.capacity) {
          a.table[(int64_t)s * mp + L / P] = np;
          a.batch_table[brow + L / P] = np;
          r.ref[np] = 1;
          const int k = atomicAdd(&s_ncow, 1);
          s_cow_src[k] = tail;
          s_cow_dst[k] = np;
        } else {
          atomicOr(r.err, kArenaCorrupt);
        }
      }
      for (int p = oldp; p < newp; ++p) {
        const int np = r.stack[pos--];
        const int id = np >= 0 && np < a.capacity ? np : -1;
        if (id < 0) atomicOr(r.err, kArenaCorrupt);
        else r.ref[id] = 1;
        a.table[(int64_t)s * mp + p] = id;
        a.batch_table[brow + p] = id;
      }
      a.lens[s] = nl;
    } else if (s >= 0 && blocked && w > 0) {
      // no page for the new tokens in the batch row: from the one the first goes to
      for (int p = L / P; p < min(mp, cdiv(L + w, P)); ++p) a.batch_table[brow + p] = -1;
    }
    if (i < a.count) {
      // A row that cannot grow reports length 0: a single-token append puts
      // its token at lens - 1, which for the old length L would be the last
      // cached token (a valid, possibly shared page when L % P == 0).  With 0
      // the append writes nothing and the attention reads nothing; the host
      // raises on the error bit and discards the step's output.
      a.batch_starts[i] = L;
      a.batch_lens[i] = blocked && w > 0 ? 0 : nl;
    }
    __syncthreads();
    if (threadIdx.x == 0 && !s_fail) s_top = top - total;
    // copy-on-write: the shared tail's bytes into the new page, in every layer's pool
    const int64_t vecs = a.page_bytes / 16;
    for (int k = 0; k < s_ncow; ++k)
      for (int l = 0; l < a.num_pools; ++l) {
        const u4 *src = (const u4 *)(a.pools[l] + (int64_t)s_cow_src[k] * a.page_bytes);
        u4 *dst = (u4 *)(a.pools[l] + (int64_t)s_cow_dst[k] * a.page_bytes);
        for (int64_t v = threadIdx.x; v < vecs; v += kThreads) dst[v] = src[v];
      }
    __syncthreads();  // s_top and LDS reuse by the next chunk
  }
  if (threadIdx.x == 0) *r.top = s_top;
}

// Per-item page ranges [from, to) of `count` items, flattened over the
// workgroup: calls f(item, page index) for every page of every item.
template <typename F>
__device__ __forceinline__ void for_each_page(const int *s_from, const int *s_to, int n, int *s_wave,
                                              int *s_base, F f) {
  const int t = threadIdx.x;
  const int len = t < n ? s_to[t] - s_from[t] : 0;
  int total;
  const int incl = block_scan_incl(len, s_wave, &total);
  s_base[t] = incl - len;
  __syncthreads();
  for (int e = t; e < total; e += kThreads) {
    int lo = 0, hi = n - 1;  // the last item whose base <= e
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_base[mid] <= e) lo = mid; else hi = mid - 1;
    }
    f(lo, s_from[lo] + (e - s_base[lo]));
  }
  __syncthreads();
}

// Truncate slots to arg[i] tokens (0 releases the slot's pages); pages whose
// last reference goes back on the free stack.
__global__ __launch_bounds__(kThreads) void arena_release_kernel(ArenaArgs a) {
  __shared__ int s_wave[kWaves];
  __shared__ int s_slot[kThreads], s_from[kThreads], s_to[kThreads], s_base[kThreads];
  __shared__ int s_top, s_freed;
  const ArenaRefs r(a);
  const int P = a.page_tokens, mp = a.max_pages;
  if (threadIdx.x == 0) { s_top = *r.top; s_freed = 0; }
  for (int c0 = 0; c0 < a.count; c0 += kThreads) {
    const int i = c0 + threadIdx.x;
    int s = -1, from = 0, to = 0;
    if (i < a.count) {
      s = a.slots[i];
      const int keep = a.arg[i];
      if (s < 0 || s >= a.num_slots) {
        atomicOr(r.err, kArenaBadArgument);
        s = -1;
      } else {
        const int L = a.lens[s];
        if (keep < 0 || keep > L) {
          atomicOr(r.err, kArenaBadArgument);
          s = -1;
        } else {
          from = cdiv(keep, P);
          to = cdiv(L, P);
          a.lens[s] = keep;
        }
      }
    }
    s_slot[threadIdx.x] = s;
    s_from[threadIdx.x] = s >= 0 ? from : 0;
    s_to[threadIdx.x] = s >= 0 ? to : 0;
    __syncthreads();
    const int n = min(kThreads, a.count - c0);
    for_each_page(s_from, s_to, n, s_wave, s_base, [&](int item, int p) {
      int32_t *entry = a.table + (int64_t)s_slot[item] * mp + p;
      const int id = *entry;
      *entry = -1;
      if (id < 0 || id >= a.capacity) {
        atomicOr(r.err, kArenaCorrupt);
        return;
      }
      const int before = atomicSub(&r.ref[id], 1);
      if (before == 1) {
        const int k = atomicAdd(&s_freed, 1);
        if (s_top + k < a.capacity) r.stack[s_top + k] = id;
        else atomicOr(r.err, kArenaCorrupt);
      } else if (before < 1) {
        atomicOr(r.err, kArenaCorrupt);
      }
    });
  }
  if (threadIdx.x == 0) *r.top = min(s_top + s_freed, a.capacity);
}

// Fork: slot arg[i] (empty) becomes a copy of slot slots[i] sharing its pages.
__global__ __launch_bounds__(kThreads) void arena_fork_kernel(ArenaArgs a) {
  __shared__ int s_wave[kWaves];
  __shared__ int s_src[kThreads], s_dst[kThreads], s_from[kThreads], s_to[kThreads], s_base[kThreads];
  const ArenaRefs r(a);
  const int P = a.page_tokens, mp = a.max_pages;
  for (int c0 = 0; c0 < a.count; c0 += kThreads) {
    const int i = c0 + threadIdx.x;
    int src = -1, dst = -1, n = 0;
    if (i < a.count) {
      src = a.slots[i];
      dst = a.arg[i];
      if (src < 0 || src >= a.num_slots || dst < 0 || dst >= a.num_slots || src == dst ||
          a.lens[dst] != 0) {
        atomicOr(r.err, kArenaBadArgument);
        src = dst = -1;
      } else {
        n = cdiv(a.lens[src], P);
      }
    }
    s_src[threadIdx.x] = src;
    s_dst[threadIdx.x] = dst;
    s_from[threadIdx.x] = 0;
    s_to[threadIdx.x] = n;
    __syncthreads();
    const int items = min(kThreads, a.count - c0);
    for_each_page(s_from, s_to, items, s_wave, s_base, [&](int item, int p) {
      const int id = a.table[(int64_t)s_src[item] * mp + p];
      a.table[(int64_t)s_dst[item] * mp + p] = id;
      if (id >= 0 && id < a.capacity) atomicAdd(&r.ref[id], 1);
      else atomicOr(r.err, kArenaCorrupt);
    });
    if (dst >= 0) a.lens[dst] = a.lens[src];
    __syncthreads();
  }
}

}  // namespace

hipError_t launch_arena_init(hipStream_t stream, int32_t *state, int capacity) {
  const int64_t n = capacity > kArenaHeaderWords ? capacity : kArenaHeaderWords;
  hipLaunchKernelGGL(arena_init_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, state,
                     capacity);
  return hipGetLastError();
}

hipError_t launch_arena(hipStream_t stream, ArenaOp op, const ArenaArgs &a) {
  if (a.count <= 0) return hipSuccess;
  switch (op) {
    case ArenaOp::Reserve:
      hipLaunchKernelGGL(arena_reserve_kernel, dim3(1), dim3(kThreads), 0, stream, a);
      break;
    case ArenaOp::Release:
      hipLaunchKernelGGL(arena_release_kernel, dim3(1), dim3(kThreads), 0, stream, a);
      break;
    case ArenaOp::Fork:
      hipLaunchKernelGGL(arena_fork_kernel, dim3(1), dim3(kThreads), 0, stream, a);
      break;
  }
  return hipGetLastError();
}

}  // namespace pkv
