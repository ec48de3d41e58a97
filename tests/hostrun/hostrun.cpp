// The runtime of the host build of the kernels (see hip/hip_runtime.h): workgroups run one after another, their
// threads as fibers switched by a few instructions of x86-64 (callee-saved registers and the stack pointer), cross-lane
// operations and barriers completed when the last thread of the wave / workgroup reaches them.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <sys/mman.h>
#include <unistd.h>

#include <vector>

#include "hip/hip_runtime.h"

extern "C" void hostrun_switch(void** save_sp, void* next_sp);
asm(R"(
  .text
  .globl hostrun_switch
  .type hostrun_switch, @function
hostrun_switch:
  pushq %rbp
  pushq %rbx
  pushq %r12
  pushq %r13
  pushq %r14
  pushq %r15
  movq %rsp, (%rdi)
  movq %rsi, %rsp
  popq %r15
  popq %r14
  popq %r13
  popq %r12
  popq %rbx
  popq %rbp
  ret
  .size hostrun_switch, .-hostrun_switch
)");

namespace hostrun {

Fiber* cur = nullptr;
Idx3 block_idx{0, 0, 0}, block_dim{1, 1, 1}, grid_dim{1, 1, 1};

namespace {

constexpr size_t STACK = 512 * 1024;  // a fiber's stack (a guard page below it)
constexpr size_t GUARD = 4096;

struct Launch {
  const char* name = "";
  const std::function<void()>* body = nullptr;
  std::vector<Fiber> fibers;
  std::vector<Wave> waves;
  int live = 0, at_barrier = 0;
  void* sched_sp = nullptr;
  unsigned char* lds = nullptr;
  size_t lds_bytes = 0;
};

Launch L;
std::vector<char*> stacks;  // reused from launch to launch
std::vector<unsigned char> lds_store;
int g_error = 0;

char* stack_of(size_t i) {
  while (stacks.size() <= i) {
    void* p = mmap(nullptr, STACK + GUARD, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
    if (p == MAP_FAILED) die("no memory for a fiber stack");
    mprotect(p, GUARD, PROT_NONE);
    stacks.push_back((char*)p + GUARD);
  }
  return stacks[i];
}

void release_barrier() {
  for (Fiber& f : L.fibers)
    if (f.at_barrier) {
      f.at_barrier = false;
      f.state = READY;
    }
  L.at_barrier = 0;
}

void thread_exit(Fiber* f) {
  f->state = DONE;
  --L.live;
  Wave& w = *f->wave;
  w.live &= ~(1ull << f->lane);
  w.arrived &= ~(1ull << f->lane);
  if (w.arrived && w.arrived == w.live) complete(w);
  if (L.at_barrier && L.at_barrier == L.live) release_barrier();
}

[[noreturn]] void fiber_main() {
  (*L.body)();
  Fiber* f = cur;
  thread_exit(f);
  void* dummy;
  hostrun_switch(&dummy, L.sched_sp);
  __builtin_unreachable();
}

void start_fiber(Fiber& f, size_t i) {
  f.stack = stack_of(i);
  uintptr_t top = ((uintptr_t)f.stack + STACK) & ~(uintptr_t)15;
  void** sp = (void**)top;
  *--sp = nullptr;                      // the slot the entry sees as its return address: rsp % 16 == 8 at entry
  *--sp = (void*)&fiber_main;           // popped by ret
  for (int r = 0; r < 6; ++r) *--sp = nullptr;  // rbp rbx r12 r13 r14 r15
  f.sp = sp;
  f.state = READY;
  f.at_barrier = false;
}

void deadlock() {
  fprintf(stderr, "hostrun: %s, block (%u, %u, %u): every live thread waits\n", L.name, block_idx.x, block_idx.y,
          block_idx.z);
  for (size_t w = 0; w < L.waves.size(); ++w) {
    int bar = 0;
    for (int l = 0; l < 64; ++l) {
      size_t i = w * 64 + l;
      if (i < L.fibers.size() && L.fibers[i].at_barrier) ++bar;
    }
    fprintf(stderr, "  wave %zu: live %016llx, at a cross-lane operation %016llx, at the barrier %d\n", w,
            (unsigned long long)L.waves[w].live, (unsigned long long)L.waves[w].arrived, bar);
  }
  die("deadlock");
}

}  // namespace

void die(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  fprintf(stderr, "hostrun: ");
  vfprintf(stderr, fmt, ap);
  fprintf(stderr, " (kernel %s, block %u %u %u, thread %d)\n", L.name, block_idx.x, block_idx.y, block_idx.z,
          cur ? cur->flat : -1);
  va_end(ap);
  fflush(stderr);
  abort();
}

void yield() { hostrun_switch(&cur->sp, L.sched_sp); }

void complete(Wave& w) {
  w.pending(w, w.pending_fn);
  const uint64_t arrived = w.arrived;
  w.arrived = 0;
  w.pending = nullptr;
  const size_t base = (size_t)(&w - L.waves.data()) * 64;
  for (int l = 0; l < 64; ++l)
    if ((arrived >> l) & 1) L.fibers[base + l].state = READY;
}

void barrier() {
  Fiber* f = cur;
  if (f->wave->arrived) die("a barrier while lanes of the wave wait at a cross-lane operation");
  f->at_barrier = true;
  ++L.at_barrier;
  if (L.at_barrier == L.live) {
    release_barrier();
    return;
  }
  f->state = WAITING;
  yield();
}

unsigned char* lds_base() { return L.lds; }
size_t lds_size() { return L.lds_bytes; }

uint32_t lds_addr(const void* p) {
  const uintptr_t a = (uintptr_t)p, b = (uintptr_t)L.lds;
  if (a < b || a > b + L.lds_bytes) die("an LDS address of memory outside the dynamic LDS");
  return (uint32_t)(a - b);
}

void load_lds(const void* src, uint32_t m0) {
  // a direct load of 16 bytes a lane: lane l's bytes land at M0 + 16 l
  const size_t at = (size_t)m0 + 16 * (size_t)cur->lane;
  if (at + 16 > L.lds_bytes)
    die("a direct load into LDS at %zu, past the dynamic LDS of %zu bytes", at, L.lds_bytes);
  if (at + 16 > 128 * 1024) die("a direct load into LDS at %zu, at or above 128 KiB", at);
  memcpy(L.lds + at, src, 16);
}

// HOSTRUN_SEED=<n>: the workgroups of a launch in a shuffled order, and in every scheduling pass the waves of a
// workgroup in a shuffled order (a wave's lanes stay in order): a kernel whose waves share LDS without a barrier
// between the write and the read, or whose result depends on which workgroup finishes last, gives different
// results from seed to seed
struct Shuffle {
  uint64_t state = 0;
  bool on = false;
  Shuffle() {
    if (const char* e = getenv("HOSTRUN_SEED")) {
      on = true;
      state = 0x9e3779b97f4a7c15ull ^ strtoull(e, nullptr, 10);
    }
  }
  uint64_t next() {  // xorshift64*
    state ^= state >> 12;
    state ^= state << 25;
    state ^= state >> 27;
    return state * 0x2545f4914f6cdd1dull;
  }
  template <class V> void apply(V& v) {
    if (!on) return;
    for (size_t i = v.size(); i > 1; --i) std::swap(v[i - 1], v[next() % i]);
  }
};

void launch(const char* name, dim3 grid, dim3 block, size_t shmem, const std::function<void()>& body) {
  static Shuffle shuffle;
  const size_t n = (size_t)block.x * block.y * block.z;
  if (n == 0 || n > 1024) die("a workgroup of %zu threads", n);
  if ((size_t)grid.x * grid.y * grid.z == 0) die("an empty grid");
  if (shmem > 160 * 1024) die("%zu bytes of dynamic LDS", shmem);
  L.name = name;
  L.body = &body;
  L.fibers.assign(n, Fiber{});
  L.waves.assign((n + 63) / 64, Wave{});
  lds_store.assign(shmem + 16, 0);
  L.lds = lds_store.data();
  L.lds_bytes = shmem;
  block_dim = Idx3{block.x, block.y, block.z};
  grid_dim = Idx3{grid.x, grid.y, grid.z};
  std::vector<Idx3> order;
  order.reserve((size_t)grid.x * grid.y * grid.z);
  for (uint32_t bz = 0; bz < grid.z; ++bz)
    for (uint32_t by = 0; by < grid.y; ++by)
      for (uint32_t bx = 0; bx < grid.x; ++bx) order.push_back(Idx3{bx, by, bz});
  shuffle.apply(order);
  const size_t n_waves = (n + 63) / 64;
  std::vector<size_t> wave_order(n_waves);
  for (size_t w = 0; w < n_waves; ++w) wave_order[w] = w;
  for (const Idx3& b : order) {
        block_idx = b;
        memset(L.lds, 0xa5, shmem);  // what the previous workgroup left: nothing to rely on
        for (Wave& w : L.waves) {
          w.live = w.arrived = 0;
          w.pending = nullptr;
        }
        for (size_t i = 0; i < n; ++i) {
          Fiber& f = L.fibers[i];
          f.flat = (int)i;
          f.tid = Idx3{(uint32_t)(i % block.x), (uint32_t)(i / block.x % block.y), (uint32_t)(i / block.x / block.y)};
          f.lane = (int)(i % 64);
          f.wave = &L.waves[i / 64];
          f.wave->live |= 1ull << f.lane;
          start_fiber(f, i);
        }
        L.live = (int)n;
        L.at_barrier = 0;
        for (;;) {
          bool ran = false;
          shuffle.apply(wave_order);
          for (size_t w : wave_order)
            for (size_t i = w * 64; i < std::min(n, w * 64 + 64); ++i) {
              Fiber& f = L.fibers[i];
              if (f.state != READY) continue;
              cur = &f;
              hostrun_switch(&L.sched_sp, f.sp);
              ran = true;
            }
          if (L.live == 0) break;
          if (!ran) deadlock();
        }
        cur = nullptr;
      }
}

}  // namespace hostrun

using namespace hostrun;

static int g_cus = 0;

hipError_t hipGetLastError() {
  int e = hostrun::g_error;
  hostrun::g_error = 0;
  return e;
}
const char* hipGetErrorString(hipError_t e) { return e ? "host build error" : "no error"; }
hipError_t hipGetDevice(int* dev) {
  *dev = 0;
  return hipSuccess;
}
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t, int) {
  if (!g_cus) {
    const char* e = getenv("HOSTRUN_CUS");
    g_cus = e ? atoi(e) : 256;
    if (g_cus <= 0) g_cus = 256;
  }
  *v = g_cus;
  return hipSuccess;
}
hipError_t hipMemcpyAsync(void* dst, const void* src, size_t n, hipMemcpyKind, hipStream_t) {
  memmove(dst, src, n);
  return hipSuccess;
}
hipError_t hipMemsetAsync(void* dst, int v, size_t n, hipStream_t) {
  memset(dst, v, n);
  return hipSuccess;
}
hipError_t hipFuncGetAttributes(hipFuncAttributes* a, const void*) {
  a->sharedSizeBytes = 0;
  return hipSuccess;
}
int hostrun_occupancy(int threads, size_t shmem) {
  // a CU holds 32 waves and 160 KiB of LDS
  int n = 32 / std::max(1, (threads + 63) / 64);
  if (shmem) n = std::min<int>(n, (int)(160 * 1024 / shmem));
  return std::max(1, n);
}
