// Checks the C++ runtime wrapper (include/xpu_runtime.hpp) against the
// contract of the class it stands in for, qwen3::LevelZeroRuntime
// (qwen3/level_zero_runtime.hpp:18-48, level_zero_runtime.cpp:163-255):
// device queries, the memory reserve check, aligned runtime-owned
// allocations, synchronous copies, launch by entry-name fragment with its
// ambiguity and argument errors rethrown as std::runtime_error, and a chain
// of three blocking launches (Embedding -> RmsNorm -> Argmax) whose answer is
// known in closed form. Prints "runtime contract: PASS" and returns 0, or
// names the first failed check and returns 1.
#include "xpu_runtime.hpp"

#include <cstdint>
#include <cstring>
#include <iostream>
#include <string>
#include <vector>

namespace {

int failures = 0;

void expect(bool ok, const std::string &what) {
  if (!ok) {
    std::cerr << "FAILED: " << what << '\n';
    ++failures;
  }
}

// runs f and reports whether it threw std::runtime_error whose text holds `needle`
template <typename F> bool throws_with(F &&f, const std::string &needle) {
  try {
    f();
  } catch (const std::runtime_error &e) {
    return std::string(e.what()).find(needle) != std::string::npos;
  }
  return false;
}

uint16_t bf16_of_small_int(int v) {  // exact for |v| < 256
  float f = static_cast<float>(v);
  uint32_t bits;
  std::memcpy(&bits, &f, 4);
  return static_cast<uint16_t>(bits >> 16);
}

}  // namespace

int main() {
  try {
    xpu::HipRuntime rt("");
    expect(!rt.device_name().empty(), "device_name() is empty");
    expect(rt.device_memory() > (1ull << 30), "device_memory() below 1 GiB");
    rt.require_device_and_memory(64ull << 20);
    expect(throws_with([&] { rt.require_device_and_memory(rt.device_memory()); }, "memory"),
           "a request for all device memory passes the 512 MiB reserve check");

    for (uint64_t align : {uint64_t{256}, uint64_t{1024}, uint64_t{4096}}) {
      void *p = rt.allocate_device(1000, align);
      expect(reinterpret_cast<uintptr_t>(p) % align == 0, "allocation not aligned to " + std::to_string(align));
    }
    expect(throws_with([&] { rt.allocate_device(1000, 3000); }, "alignment"), "a non-power-of-two alignment passes");

    // synchronous round trip of a byte pattern
    std::vector<uint8_t> bytes(1 << 20), back(bytes.size());
    for (size_t i = 0; i < bytes.size(); ++i) bytes[i] = static_cast<uint8_t>((i * 2654435761u) >> 13);
    void *buf = rt.allocate_device(bytes.size());
    rt.copy_to_device(buf, bytes.data(), bytes.size());
    rt.copy_from_device(back.data(), buf, back.size());
    expect(bytes == back, "copy_to_device / copy_from_device round trip differs");

    // fragment lookup: "Qwen" names all eight entries, "NoSuchEntry" none
    const uint32_t width = 640;
    void *out = rt.allocate_device(width * 2);
    expect(throws_with([&] { rt.launch("Qwen", 1, {}); }, "ambiguous"), "an ambiguous fragment launches");
    expect(throws_with([&] { rt.launch("NoSuchEntry", 1, {}); }, "NoSuchEntry"), "an unknown fragment launches");
    expect(throws_with([&] { rt.launch("Argmax", 1, {xpu::kernel_argument(out)}); }, "argument"),
           "a launch with too few arguments is accepted");
    expect(throws_with([&] { rt.launch("NoSuchEntry", 1, {}); }, "xpu_rt_launch(") &&
               throws_with([&] { rt.launch("NoSuchEntry", 1, {}); }, " failed at "),
           "errors do not name the failing call and its location");

    // Embedding -> RmsNorm -> Argmax, each launch blocking: row t of the
    // table holds small integers whose unique maximum sits at (37 t) mod
    // width; unit gains keep RMSNorm monotonic, so the argmax is that index.
    const uint32_t vocab = 24, token = 17;
    std::vector<uint16_t> table(static_cast<size_t>(vocab) * width), gains(width, bf16_of_small_int(1));
    for (uint32_t t = 0; t < vocab; ++t)
      for (uint32_t i = 0; i < width; ++i)
        table[t * width + i] = bf16_of_small_int(i == (37 * t) % width ? 100 : static_cast<int>((i * 7 + t) % 64) - 32);
    void *d_table = rt.allocate_device(table.size() * 2), *d_gains = rt.allocate_device(width * 2);
    void *d_norm = rt.allocate_device(width * 2), *d_token = rt.allocate_device(4);
    rt.copy_to_device(d_table, table.data(), table.size() * 2);
    rt.copy_to_device(d_gains, gains.data(), width * 2);
    const float eps = 1e-6f;
    rt.launch("Embedding", width,
              {xpu::kernel_argument(d_table), xpu::kernel_argument(out), xpu::kernel_argument(token),
               xpu::kernel_argument(width)});
    rt.launch("RmsNorm", 1,
              {xpu::kernel_argument(out), xpu::kernel_argument(d_gains), xpu::kernel_argument(d_norm),
               xpu::kernel_argument(width), xpu::kernel_argument(eps)});
    rt.launch("Argmax", 1, {xpu::kernel_argument(d_norm), xpu::kernel_argument(d_token), xpu::kernel_argument(width)});
    uint32_t got = 0;
    rt.copy_from_device(&got, d_token, 4);
    expect(got == (37 * token) % width,
           "Embedding -> RmsNorm -> Argmax gave " + std::to_string(got) + ", expected " +
               std::to_string((37 * token) % width));
    std::vector<uint16_t> row(width);
    rt.copy_from_device(row.data(), out, width * 2);
    expect(std::equal(row.begin(), row.end(), table.begin() + token * width), "Embedding row differs from the table");
  } catch (const std::exception &e) {
    std::cerr << "FAILED: unexpected exception: " << e.what() << '\n';
    return 1;
  }
  if (failures) return 1;
  std::cout << "runtime contract: PASS\n";
  return 0;
}
