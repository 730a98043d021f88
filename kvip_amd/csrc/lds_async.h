// LDS access around in-flight direct-to-LDS loads (global_load_lds_dwordx4).
//
// LLVM's wait insertion cannot tell an LDS read apart from the LDS bytes a pending
// direct-to-LDS load will write, so it puts s_waitcnt vmcnt(0) in front of every LDS
// read while such a load is in flight. That drains every prefetch before each read and
// defeats multi-buffering. Kernels that stream K through LDS therefore issue their LDS
// accesses as inline asm, which that pass does not track:
//   * a read helper issues its ds_read(s) and waits lgkmcnt(0) in the same asm block, so
//     the output registers are valid when the block ends (no uninitialised copies);
//   * stores and atomics are fire-and-forget; LDS operations of one wave execute in issue
//     order, so a later read of the same wave sees them;
//   * the kernel waits for its own direct-to-LDS loads with an explicit vmcnt(N): vector
//     memory operations complete in issue order, and N counts the vector memory
//     instructions issued after the load being waited for.
#pragma once

#include "kvip_device.h"

#define LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

namespace kvip {

typedef int v2i __attribute__((ext_vector_type(2)));

KVIP_DEVICE uint32_t lds_addr(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(LDS_PTR(p)));
}

// The four 16-byte K fragment pieces of a tile row and one 4-byte value (the row's key
// scale), then wait for them.
KVIP_DEVICE void lds_read_tile(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, uint32_t as, v4i (&kb)[4],
                               float& ks) {
    asm volatile(
        "ds_read_b128 %0, %5\n"
        "ds_read_b128 %1, %6\n"
        "ds_read_b128 %2, %7\n"
        "ds_read_b128 %3, %8\n"
        "ds_read_b32 %4, %9\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(kb[0]), "=&v"(kb[1]), "=&v"(kb[2]), "=&v"(kb[3]), "=&v"(ks)
        : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "v"(as));
}

// The eight 16-byte K fragment pieces of a bf16 tile row (addresses a[u] + off) and its key
// scale, then wait for them.
KVIP_DEVICE void lds_read_tile8(const uint32_t (&a)[8], uint32_t off, uint32_t as, v4i (&kb)[8], float& ks) {
    asm volatile(
        "ds_read_b128 %0, %9\n"
        "ds_read_b128 %1, %10\n"
        "ds_read_b128 %2, %11\n"
        "ds_read_b128 %3, %12\n"
        "ds_read_b128 %4, %13\n"
        "ds_read_b128 %5, %14\n"
        "ds_read_b128 %6, %15\n"
        "ds_read_b128 %7, %16\n"
        "ds_read_b32 %8, %17\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(kb[0]), "=&v"(kb[1]), "=&v"(kb[2]), "=&v"(kb[3]), "=&v"(kb[4]), "=&v"(kb[5]), "=&v"(kb[6]),
          "=&v"(kb[7]), "=&v"(ks)
        : "v"(a[0] + off), "v"(a[1] + off), "v"(a[2] + off), "v"(a[3] + off), "v"(a[4] + off), "v"(a[5] + off),
          "v"(a[6] + off), "v"(a[7] + off), "v"(as));
}

KVIP_DEVICE v2i lds_read_b64(uint32_t a) {
    v2i v;
    asm volatile("ds_read_b64 %0, %1\ns_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(a));
    return v;
}

KVIP_DEVICE uint32_t lds_read_b32(uint32_t a) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1\ns_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(a));
    return v;
}

KVIP_DEVICE void lds_write_b16(uint32_t a, uint32_t v) { asm volatile("ds_write_b16 %0, %1" : : "v"(a), "v"(v)); }

KVIP_DEVICE void lds_write_b32(uint32_t a, uint32_t v) { asm volatile("ds_write_b32 %0, %1" : : "v"(a), "v"(v)); }

KVIP_DEVICE void lds_add_u32(uint32_t a, uint32_t v) { asm volatile("ds_add_u32 %0, %1" : : "v"(a), "v"(v)); }

KVIP_DEVICE v4i lds_read_b128(uint32_t a) {
    v4i v;
    asm volatile("ds_read_b128 %0, %1\ns_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(a));
    return v;
}

KVIP_DEVICE void lds_write_b128(uint32_t a, v4i v) { asm volatile("ds_write_b128 %0, %1" : : "v"(a), "v"(v)); }

// Waits until at most N vector memory instructions of this wave are outstanding (N is a
// compile-time count, 0..63).
template <int N>
KVIP_DEVICE void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit count");
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// Workgroup barrier after this wave's LDS operations and all but its `stores` most recent
// vector memory instructions (0, 1 or 2) have completed.
KVIP_DEVICE void lds_barrier(int stores) {
    if (stores >= 2) {
        asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)" : : : "memory");
    } else if (stores == 1) {
        asm volatile("s_waitcnt vmcnt(1) lgkmcnt(0)" : : : "memory");
    } else {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" : : : "memory");
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" : : : "memory");
}

}  // namespace kvip
