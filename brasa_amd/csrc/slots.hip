// Per-stream slots of the library's device-side launch state (host code only).
//
// The split merges of decode and prefill count arrivals in counters the library owns (device
// arrays, zero at load, returned to zero by every launch). Two launches in flight at the same
// time must not share counters. Launches on one stream run in order, so each stream gets a slot
// of its own: the first use of a (device, stream) pair assigns the next free slot, and the pair
// keeps it until brasa_release_workspaces(). hipStreamPerThread names a different stream in
// every host thread, so for it the thread is part of the key.
#include <atomic>
#include <cstdint>
#include <mutex>
#include <thread>

#include "common.hpp"

namespace brasa {

namespace {

struct SlotKey {
    uintptr_t stream = 0;
    size_t thread = 0;  // hipStreamPerThread only
    bool used = false;
};

std::mutex g_slot_mu;
SlotKey g_slot_keys[kMaxDevices][kStreamSlots];
// Bumped by release_stream_slots(); a thread's cached lookup is valid for one generation.
std::atomic<unsigned> g_slot_gen{1};

struct SlotCache {
    int dev = -1;
    uintptr_t stream = 0;
    unsigned gen = 0;
    int slot = -1;
};
thread_local SlotCache t_slot_cache;

}  // namespace

// The slot of `stream` on device `dev` (0 <= dev < kMaxDevices), assigned on first use; -1 when
// the device's slots are all taken.
int slot_lookup(int dev, hipStream_t stream) {
    const uintptr_t key = reinterpret_cast<uintptr_t>(stream);
    const unsigned gen = g_slot_gen.load(std::memory_order_acquire);
    SlotCache& c = t_slot_cache;
    if (c.dev == dev && c.stream == key && c.gen == gen) return c.slot;
    const size_t thread = stream == hipStreamPerThread
                              ? std::hash<std::thread::id>()(std::this_thread::get_id())
                              : 0;
    int slot = -1;
    {
        std::lock_guard<std::mutex> lock(g_slot_mu);
        int free_slot = -1;
        for (int i = 0; i < kStreamSlots; ++i) {
            const SlotKey& k = g_slot_keys[dev][i];
            if (k.used && k.stream == key && k.thread == thread) {
                slot = i;
                break;
            }
            if (!k.used && free_slot < 0) free_slot = i;
        }
        if (slot < 0 && free_slot >= 0) {
            g_slot_keys[dev][free_slot] = SlotKey{key, thread, true};
            slot = free_slot;
        }
    }
    // (-1: every slot is taken; the callers then use launch plans that need no counters)
    c = SlotCache{dev, key, gen, slot};
    return slot;
}

int stream_slot(hipStream_t stream, int* dev_out, int* slot_out) {
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(BRASA_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return set_error(BRASA_ERR_LAUNCH, "device %d out of range", dev);
    *dev_out = dev;
    *slot_out = slot_lookup(dev, stream);
    return BRASA_OK;
}

void release_stream_slots() {
    std::lock_guard<std::mutex> lock(g_slot_mu);
    for (auto& dev : g_slot_keys)
        for (auto& k : dev) k = SlotKey{};
    g_slot_gen.fetch_add(1, std::memory_order_acq_rel);
}

}  // namespace brasa

extern "C" int brasa_test_stream_slot(int device, void* stream, int* slot) {
    using namespace brasa;
    if (device < 0 || device >= kMaxDevices || !slot)
        return set_error(BRASA_ERR_ARG, "stream slot: device %d", device);
    *slot = slot_lookup(device, static_cast<hipStream_t>(stream));
    return BRASA_OK;
}
