// The host side of the HIP stand-in in include/hip/hip_runtime.h: lane fibers,
// wave and block rendezvous, the per-wave vector-memory queue, launches, and the
// memory checks.  Test infrastructure only.
//
// A block's threads are fibers on one host thread.  A fiber runs until it
// reaches a rendezvous (a cross-lane operation of its wave, or a block barrier)
// and then yields; the scheduler resumes the block's runnable fibers in thread
// order.  A cross-lane operation completes when every live lane of the wave has
// posted its input; inputs sit in one of two slot banks by the parity of the
// wave's operation count, so a lane that runs ahead to the next operation does
// not overwrite what the others still read.
#include "hip/hip_runtime.h"

#include <chrono>
#include <cstdarg>
#include <deque>
#include <dlfcn.h>
#include <link.h>
#include <sys/mman.h>
#include <vector>

thread_local emu_uint3 threadIdx, blockIdx, blockDim, gridDim;

extern "C" void* __asan_region_is_poisoned(void* beg, size_t size) __attribute__((weak));
extern "C" void __sanitizer_start_switch_fiber(void** fake_stack_save, const void* bottom, size_t size)
    __attribute__((weak));
extern "C" void __sanitizer_finish_switch_fiber(void* fake_stack_save, const void** bottom_old,
                                                size_t* size_old) __attribute__((weak));

// void emu_switch(void** save_sp, void* load_sp): callee-saved registers and the
// floating-point control words on the current stack, its stack pointer saved,
// the other fiber's restored
asm(R"(
  .text
  .globl emu_switch
  .type emu_switch, @function
emu_switch:
  pushq %rbp
  pushq %rbx
  pushq %r12
  pushq %r13
  pushq %r14
  pushq %r15
  subq $8, %rsp
  stmxcsr (%rsp)
  fnstcw 4(%rsp)
  movq %rsp, (%rdi)
  movq %rsi, %rsp
  ldmxcsr (%rsp)
  fldcw 4(%rsp)
  addq $8, %rsp
  popq %r15
  popq %r14
  popq %r13
  popq %r12
  popq %rbx
  popq %rbp
  ret
  .size emu_switch, .-emu_switch
)");
extern "C" void emu_switch(void** save_sp, void* load_sp);

namespace emu {
namespace {

constexpr size_t kMaxLds = 160 * 1024;
constexpr size_t kStack = 1 << 20;
constexpr int kSlot = 128;
alignas(4096) unsigned char g_lds[kMaxLds + 4096];

struct VmOp {
  struct Copy {
    const unsigned char* src;   // null: zeros
    unsigned char* dst;
    int size;
  };
  std::vector<Copy> copies;
};

enum State { RUNNABLE, WAIT_WAVE, WAIT_BLOCK, DONE };

struct Fiber {
  void* sp = nullptr;
  unsigned char* stack = nullptr;
  State state = RUNNABLE;
  int tid = 0;
  uint64_t wave_ops = 0;       // cross-lane operations this lane has posted
};

struct Wave {
  int live = 64, arrived = 0;
  alignas(64) unsigned char slot[2][64][kSlot];
  std::deque<VmOp> vm;
};

struct Block {
  int nthreads = 0, live = 0, arrived = 0;
  std::vector<Fiber> fibers;
  std::vector<int> orv;
  Wave waves[16];
  size_t lds_bytes = 0;
  void* sched_sp = nullptr;
  void* body_ctx = nullptr;
  void (*body)(void*) = nullptr;
  dim3 grid, block;
  unsigned bx = 0, by = 0, bz = 0;
  std::vector<const void*> shared;     // static LDS arrays filled this block
};

thread_local Block* t_block = nullptr;
thread_local Fiber* t_fiber = nullptr;
uintptr_t g_static_lo = 0, g_static_hi = 0;   // this module's writable segment (static LDS)

int phdr_cb(struct dl_phdr_info* info, size_t, void*) {
  const uintptr_t probe = (uintptr_t)g_lds;
  for (int i = 0; i < info->dlpi_phnum; ++i) {
    const ElfW(Phdr)& ph = info->dlpi_phdr[i];
    if (ph.p_type != PT_LOAD) continue;
    const uintptr_t lo = info->dlpi_addr + ph.p_vaddr, hi = lo + ph.p_memsz;
    if (probe >= lo && probe < hi) {
      g_static_lo = lo;
      g_static_hi = hi;
      return 1;
    }
  }
  return 0;
}

void init_segments() {
  if (g_static_hi) return;
  dl_iterate_phdr(phdr_cb, nullptr);
  if (!g_static_hi) fail("cannot find the module's writable segment");
  if ((g_static_lo >> 32) != ((g_static_hi - 1) >> 32))
    fail("the module's data segment straddles a 4 GiB boundary: LDS addresses are not 32-bit");
}

// an LDS address (32 bits, as the kernels compute for M0) back to a pointer,
// checked to lie in the block's dynamic LDS or in the module's static data
unsigned char* lds_ptr(uint32_t a, int size) {
  const uintptr_t p = (g_static_lo & ~(uintptr_t)0xffffffffu) | a;
  const uintptr_t dyn = (uintptr_t)g_lds;
  if (p >= dyn && p + size <= dyn + t_block->lds_bytes) return (unsigned char*)p;
  if (p >= dyn && p < dyn + sizeof(g_lds))
    fail("LDS access at %#x past the launch's %zu dynamic bytes", (unsigned)(p - dyn), t_block->lds_bytes);
  if (p >= g_static_lo && p + size <= g_static_hi) return (unsigned char*)p;
  fail("LDS address %#x is not LDS", a);
  return nullptr;
}

void complete(VmOp& op) {
  for (auto& c : op.copies) {
    if (c.src) {
      check_global(c.src, c.size, "load into LDS (at completion)");
      memcpy(c.dst, c.src, c.size);
    } else {
      memset(c.dst, 0, c.size);
    }
  }
}

// SBSA_EMU_SYNC_DMA=1: loads into LDS land at issue (no check of the waits)
bool sync_dma() {
  static const bool v = getenv("SBSA_EMU_SYNC_DMA") && atoi(getenv("SBSA_EMU_SYNC_DMA"));
  return v;
}

// ---- fibers ---------------------------------------------------------------------
void yield_to_scheduler() {
  Fiber* f = t_fiber;
  void* fake = nullptr;
  if (__sanitizer_start_switch_fiber) __sanitizer_start_switch_fiber(&fake, nullptr, 0);
  emu_switch(&f->sp, t_block->sched_sp);
  if (__sanitizer_finish_switch_fiber) __sanitizer_finish_switch_fiber(fake, nullptr, nullptr);
}

[[noreturn]] void fiber_entry() {
  if (__sanitizer_finish_switch_fiber) __sanitizer_finish_switch_fiber(nullptr, nullptr, nullptr);
  Block* b = t_block;
  b->body(b->body_ctx);
  // a returned thread leaves every rendezvous
  Fiber* f = t_fiber;
  f->state = DONE;
  --b->waves[f->tid >> 6].live;
  --b->live;
  if (__sanitizer_start_switch_fiber) __sanitizer_start_switch_fiber(nullptr, nullptr, 0);
  emu_switch(&f->sp, b->sched_sp);
  abort();
}

void set_thread_ids(Block* b, int t) {
  threadIdx = emu_uint3{(unsigned)t, 0, 0};
  blockIdx = emu_uint3{b->bx, b->by, b->bz};
  blockDim = emu_uint3{b->block.x, b->block.y, b->block.z};
  gridDim = emu_uint3{b->grid.x, b->grid.y, b->grid.z};
}

// every waiting lane of a wave whose live lanes have all arrived, and every lane
// at a block barrier that all live lanes reached, becomes runnable
bool release(Block* b) {
  bool any = false;
  for (int w = 0; w < b->nthreads / 64; ++w) {
    Wave& wv = b->waves[w];
    if (wv.arrived > 0 && wv.arrived == wv.live) {
      wv.arrived = 0;
      for (int l = 0; l < 64; ++l) {
        Fiber& f = b->fibers[64 * w + l];
        if (f.state == WAIT_WAVE) f.state = RUNNABLE;
      }
      any = true;
    }
  }
  if (b->arrived > 0 && b->arrived == b->live) {
    b->arrived = 0;
    for (auto& f : b->fibers)
      if (f.state == WAIT_BLOCK) f.state = RUNNABLE;
    any = true;
  }
  return any;
}

void run_block(Block* b) {
  const int n = b->nthreads;
  b->fibers.assign(n, Fiber{});
  b->live = n;
  for (int w = 0; w < n / 64; ++w) {
    b->waves[w].live = 64;
    b->waves[w].arrived = 0;
    b->waves[w].vm.clear();
  }
  static std::vector<unsigned char*> stacks;
  while ((int)stacks.size() < n) {
    void* s = mmap(nullptr, kStack, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
    if (s == MAP_FAILED) fail("fiber stack");
    stacks.push_back(static_cast<unsigned char*>(s));
  }
  uint32_t csr[2];
  asm volatile("stmxcsr %0" : "=m"(csr[0]));
  asm volatile("fnstcw %0" : "=m"(csr[1]));
  for (int t = 0; t < n; ++t) {
    Fiber& f = b->fibers[t];
    f.tid = t;
    f.stack = stacks[t];
    // initial frame for emu_switch: the control words, six registers, then the
    // return address fiber_entry (entered with rsp % 16 == 8, as after a call)
    uint64_t* sp = reinterpret_cast<uint64_t*>(f.stack + kStack);
    *--sp = 0;
    *--sp = (uint64_t)(uintptr_t)&fiber_entry;
    for (int r = 0; r < 6; ++r) *--sp = 0;
    *--sp = (uint64_t)csr[0] | ((uint64_t)(csr[1] & 0xffff) << 32);
    f.sp = sp;
  }
  for (;;) {
    bool ran = false;
    for (int t = 0; t < n; ++t) {
      Fiber& f = b->fibers[t];
      if (f.state != RUNNABLE) continue;
      ran = true;
      t_fiber = &f;
      set_thread_ids(b, t);
      void* fake = nullptr;
      if (__sanitizer_start_switch_fiber) __sanitizer_start_switch_fiber(&fake, f.stack, kStack);
      emu_switch(&b->sched_sp, f.sp);
      if (__sanitizer_finish_switch_fiber) __sanitizer_finish_switch_fiber(fake, nullptr, nullptr);
    }
    const bool freed = release(b);
    if (b->live == 0) break;
    if (!ran && !freed) {
      int ww = 0, wb = 0;
      for (auto& f : b->fibers) {
        ww += f.state == WAIT_WAVE;
        wb += f.state == WAIT_BLOCK;
      }
      t_fiber = &b->fibers[0];
      fail("deadlock: %d lanes at a cross-lane operation, %d at a block barrier, %d live", ww, wb, b->live);
    }
  }
  t_fiber = nullptr;
}

}  // namespace

void fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  fprintf(stderr, "[emu] block (%u,%u) thread %u: ", blockIdx.x, blockIdx.y, threadIdx.x);
  vfprintf(stderr, fmt, ap);
  fprintf(stderr, "\n");
  va_end(ap);
  fflush(stderr);
  abort();
}

void shared_var(const void* p, size_t bytes) {
  Block* b = t_block;
  for (const void* q : b->shared)
    if (q == p) return;
  b->shared.push_back(p);
  memset(const_cast<void*>(p), 0xA5, bytes);
}

int lane() { return t_fiber->tid & 63; }
int wave() { return t_fiber->tid >> 6; }
void* dyn_lds() { return g_lds; }

void check_global(const void* p, size_t n, const char* what) {
  if (n == 0) return;
  if ((uintptr_t)p < 4096) fail("%s: address %p", what, p);
  if (__asan_region_is_poisoned) {
    void* bad = __asan_region_is_poisoned(const_cast<void*>(p), n);
    if (bad) fail("%s: %zu bytes at %p touch unallocated memory at %p (a GPU memory fault)", what, n, p, bad);
  }
}

const unsigned char* wave_post(const void* in, int bytes) {
  static_assert(kSlot == kSlotBytes, "slot size");
  if (bytes > kSlot) fail("wave exchange of %d bytes", bytes);
  Block* b = t_block;
  Fiber* f = t_fiber;
  Wave& w = b->waves[f->tid >> 6];
  if (w.live != 64) fail("a cross-lane operation in a wave with %d live lanes", w.live);
  const int bank = (int)(f->wave_ops & 1);
  memcpy(w.slot[bank][f->tid & 63], in, bytes);
  ++f->wave_ops;
  ++w.arrived;
  f->state = WAIT_WAVE;
  yield_to_scheduler();
  return &w.slot[bank][0][0];
}

void wave_exchange(const void* in, int bytes, void* all_out) {
  const unsigned char* bank = wave_post(in, bytes);
  unsigned char* out = static_cast<unsigned char*>(all_out);
  for (int l = 0; l < 64; ++l) memcpy(out + (size_t)l * bytes, bank + (size_t)l * kSlot, bytes);
}

void block_barrier() {
  ++t_block->arrived;
  t_fiber->state = WAIT_BLOCK;
  yield_to_scheduler();
}

int block_or(int v) {
  Block* b = t_block;
  b->orv[t_fiber->tid] = v;
  block_barrier();
  int r = 0;
  for (int i = 0; i < b->nthreads; ++i) r |= b->orv[i];
  block_barrier();
  return r != 0;
}

// buffer_load_dword{,x4} ... offen lds: lane l writes `size` bytes at M0 + size l.
// Lane 0 resumes first after the rendezvous and queues the op for the wave.
void buffer_load_lds(uint32_t rsrc[4], uint32_t lds_addr, uint32_t voffset, int size) {
  struct In {
    uint32_t r[4], lds, off;
  } in{{rsrc[0], rsrc[1], rsrc[2], rsrc[3]}, lds_addr, voffset};
  const auto all = gather(in);
  if (lane() != 0) return;
  for (int l = 1; l < 64; ++l)
    if (memcmp(all[l].r, all[0].r, 16) || all[l].lds != all[0].lds)
      fail("buffer load to LDS: resource or M0 not uniform");
  const uint64_t base = (uint64_t)all[0].r[0] | ((uint64_t)(all[0].r[1] & 0xffffu) << 32);
  const uint32_t num = all[0].r[2];
  if ((all[0].r[1] >> 16) != 0) fail("buffer load to LDS: strided resource");
  VmOp op;
  for (int l = 0; l < 64; ++l) {
    unsigned char* dst = lds_ptr(all[0].lds + (uint32_t)(size * l), size);
    const uint64_t off = all[l].off;
    const bool in_range = off + (uint64_t)size <= num;
    const unsigned char* src = in_range ? reinterpret_cast<const unsigned char*>(base + off) : nullptr;
    if (src) check_global(src, size, "buffer load to LDS (at issue)");
    op.copies.push_back({src, dst, size});
  }
  if (sync_dma()) complete(op);
  else t_block->waves[wave()].vm.push_back(std::move(op));
}

// global_load_lds: lane l loads `size` bytes from its address to lds + offset +
// size l.  The library issues some of these under a per-lane condition (legal on
// the GPU, where the wave runs them with those lanes enabled), which a
// rendezvous of all 64 lanes cannot model: each lane copies at once instead,
// and the loads are not queued (their waits are not checked).
void global_load_lds(const void* gptr, const void* lds, int size, int offset) {
  unsigned char* dst = lds_ptr((uint32_t)(uintptr_t)lds + offset + size * lane(), size);
  check_global(gptr, size, "global load to LDS");
  memcpy(dst, gptr, size);
}

// a buffer store from every lane (it counts in the wave's vector-memory queue as
// an op that has already landed)
void buffer_store(uint32_t rsrc[4], int voffset, const void* data, int size) {
  const uint64_t base = (uint64_t)rsrc[0] | ((uint64_t)(rsrc[1] & 0xffffu) << 32);
  const uint64_t off = (uint32_t)voffset;
  if (off + (uint64_t)size <= rsrc[2]) {
    void* dst = reinterpret_cast<void*>(base + off);
    check_global(dst, size, "buffer store");
    memcpy(dst, data, size);
  }
  const int dummy = 0;
  wave_post(&dummy, sizeof(int));
  if (lane() == 0) t_block->waves[wave()].vm.push_back(VmOp{});
}

// s_waitcnt: vmcnt = imm[3:0] | imm[15:14] << 4; the oldest ops land until at
// most vmcnt are outstanding (lane 0 resumes first and lands them before any
// other lane of the wave reads LDS)
void waitcnt(unsigned imm) {
  const unsigned vm = (imm & 15u) | (((imm >> 14) & 3u) << 4);
  const int dummy = 0;
  wave_post(&dummy, sizeof(int));
  if (lane() != 0) return;
  auto& q = t_block->waves[wave()].vm;
  while (q.size() > vm) {
    complete(q.front());
    q.pop_front();
  }
}

float bf16_to_float(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// SBSA_EMU_TRACE=1: one line per launch (kernel, grid, block, seconds) on stderr
void run_grid(dim3 grid, dim3 block, size_t lds, void (*body)(void*), void* ctx, const void* fn) {
  static const bool trace = getenv("SBSA_EMU_TRACE") && atoi(getenv("SBSA_EMU_TRACE"));
  const auto t0 = std::chrono::steady_clock::now();
  init_segments();
  const int nthreads = block.x * block.y * block.z;
  if (nthreads % 64 || nthreads > 1024 || block.y != 1 || block.z != 1)
    fail("launch: %d threads per block (whole waves, 1-D, at most 1024)", nthreads);
  if (lds > kMaxLds) fail("launch: %zu bytes of dynamic LDS", lds);
  Block* b = new Block();
  for (unsigned bz = 0; bz < grid.z; ++bz)
    for (unsigned by = 0; by < grid.y; ++by)
      for (unsigned bx = 0; bx < grid.x; ++bx) {
        b->nthreads = nthreads;
        b->arrived = 0;
        b->shared.clear();
        b->orv.assign(nthreads, 0);
        b->lds_bytes = lds;
        b->body = body;
        b->body_ctx = ctx;
        b->grid = grid;
        b->block = block;
        b->bx = bx;
        b->by = by;
        b->bz = bz;
        memset(g_lds, 0xA5, lds);          // stale contents: reads of unloaded LDS show
        t_block = b;
        run_block(b);
        for (int w = 0; w < nthreads / 64; ++w)
          while (!b->waves[w].vm.empty()) {
            complete(b->waves[w].vm.front());
            b->waves[w].vm.pop_front();
          }
        t_block = nullptr;
      }
  delete b;
  if (trace) {
    Dl_info info{};
    const char* name = (dladdr(fn, &info) && info.dli_sname) ? info.dli_sname : "?";
    const double s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    fprintf(stderr, "[emu] %s %p grid (%u,%u,%u) block %u lds %zu: %.3f s\n", name, fn, grid.x, grid.y,
            grid.z, block.x, lds, s);
  }
}

}  // namespace emu

extern "C" int sbsa_emu_checks_memory() { return __asan_region_is_poisoned != nullptr; }
