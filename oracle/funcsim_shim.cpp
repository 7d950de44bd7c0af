// extern "C" shim over the reference's functional simulator (runtime/src/funcsim.cpp), compiled in
// place from the reference sources into oracle/_ref -- test infrastructure only: it pins
// oracle/isa_np.py and checks the GPU device on CPU-sized programs.
#include <cstdint>
#include <cstring>
#include <exception>
#include <string>

#include "llaccel/device.h"

using llaccel::Device;
static std::string g_err;

template <class F>
static int guarded(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

extern "C" {
void* fs_create(uint64_t dram_bytes, int fusion) {
  llaccel::DeviceOptions o;
  o.dramBytes = dram_bytes;
  o.epilogueFusion = fusion != 0;
  return llaccel::makeFuncSim(o).release();
}
void* fs_create_interleaved(uint64_t dram_bytes, int fusion, uint32_t seed) {
  llaccel::DeviceOptions o;
  o.dramBytes = dram_bytes;
  o.epilogueFusion = fusion != 0;
  o.interleaveSeed = seed;
  return llaccel::makeFuncSim(o).release();
}
void fs_destroy(void* d) { delete static_cast<Device*>(d); }
int fs_write(void* d, uint64_t a, const void* s, uint64_t n) {
  return guarded([&] { static_cast<Device*>(d)->dramWrite(a, s, n); });
}
int fs_read(void* d, uint64_t a, void* dst, uint64_t n) {
  return guarded([&] { static_cast<Device*>(d)->dramRead(a, dst, n); });
}
uint64_t fs_size(void* d) { return static_cast<Device*>(d)->dramSize(); }
int fs_run(void* d, uint32_t pc, uint32_t pos, uint64_t* perf) {
  return guarded([&] {
    const auto p = static_cast<Device*>(d)->run(pc, pos);
    std::memcpy(perf, p.data(), sizeof(uint64_t) * p.size());
  });
}
int fs_sram(void* d, void* dst) {
  return guarded([&] {
    const auto s = static_cast<Device*>(d)->sramSnapshot();
    std::memcpy(dst, s.data(), s.size());
  });
}
const char* fs_error(void) { return g_err.c_str(); }
}
