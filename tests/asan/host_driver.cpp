// Host-side exercise of the C ABI for the sanitizer build (no GPU needed):
// status strings, trellis tables, layout and workspace sizes, the plan
// builder (every host-side layout, schedule and phase-block computation runs;
// only its final copy to the device fails without a GPU) and the argument
// checks of every GPU entry point.  Exits non-zero on an unexpected status.
#include "turbopress_amd.h"

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

static int failures = 0;
#define EXPECT(cond)                                                   \
  do {                                                                 \
    if (!(cond)) {                                                     \
      std::fprintf(stderr, "%s:%d: expected %s\n", __FILE__, __LINE__, #cond); \
      ++failures;                                                      \
    }                                                                  \
  } while (0)

// Stand-in device addresses: aligned, never dereferenced on the host.
static const uint8_t* fake8(uintptr_t a) { return reinterpret_cast<const uint8_t*>(a); }
static const uint16_t* fake16(uintptr_t a) { return reinterpret_cast<const uint16_t*>(a); }

static std::vector<tp_stack_linear> qwen_like(int layers) {
  // (d, n, phase in layer) of q, k, v, o, gate, up, down
  const int64_t shapes[7][3] = {{2560, 4096, 0}, {2560, 1024, 0}, {2560, 1024, 0}, {4096, 2560, 1},
                                {2560, 9728, 2}, {2560, 9728, 2}, {9728, 2560, 3}};
  std::vector<tp_stack_linear> v;
  for (int l = 0; l < layers; ++l)
    for (int j = 0; j < 7; ++j) {
      tp_stack_linear s;
      std::memset(&s, 0, sizeof(s));
      s.path_tiled = fake8(0x100000);
      s.member_tiled = fake8(0x200000);
      s.x = fake16(0x300000);
      s.ldx = shapes[j][0];
      s.rot_scale = fake16(0x400000);
      s.block = shapes[j][0] == 9728 ? 512 : (shapes[j][0] == 4096 ? 4096 : 512);
      s.scales = fake16(0x500000);
      s.bias = (j % 3 == 0) ? fake16(0x600000) : nullptr;
      s.y = reinterpret_cast<uint16_t*>(0x700000);
      s.ldy = shapes[j][1];
      s.n = shapes[j][1];
      s.d = shapes[j][0];
      s.phase = 4 * l + (int)shapes[j][2];
      v.push_back(s);
    }
  return v;
}

static void plan_cases() {
  for (int64_t batch : {1, 4, 5, 32}) {
    std::vector<tp_stack_linear> L = qwen_like(36);
    const int64_t bytes = tp_stack_plan_bytes(L.data(), (int)L.size(), 3, batch);
    EXPECT(bytes > 0);
    void* plan = std::aligned_alloc(256, (size_t)((bytes + 255) / 256 * 256));
    EXPECT(plan != nullptr);
    // the host image is built in full; the copy to a host "device" address fails
    const int st = tp_stack_plan_init(L.data(), (int)L.size(), 3, batch, plan, bytes);
    EXPECT(st != TP_OK);
    EXPECT(tp_stack_plan_init(L.data(), (int)L.size(), 3, batch, plan, bytes - 1) == TP_ERR_WORKSPACE);
    std::free(plan);
    std::vector<int64_t> ns;
    for (const auto& s : L) ns.push_back(s.n);
    EXPECT(tp_stack_plan_blocks(ns.data(), (int)ns.size()) > 0);
  }
  // many small linears, every phase distinct: 8192 linears
  {
    std::vector<tp_stack_linear> L = qwen_like(1);
    std::vector<tp_stack_linear> M;
    for (int i = 0; i < 8192; ++i) {
      tp_stack_linear s = L[i % 7];
      s.phase = i / 3;
      M.push_back(s);
    }
    const int64_t bytes = tp_stack_plan_bytes(M.data(), (int)M.size(), 2, 2);
    EXPECT(bytes > 0);
    void* plan = std::aligned_alloc(256, (size_t)((bytes + 255) / 256 * 256));
    EXPECT(tp_stack_plan_init(M.data(), (int)M.size(), 2, 2, plan, bytes) != TP_OK);
    std::free(plan);
  }
  // invalid lists
  std::vector<tp_stack_linear> L = qwen_like(2);
  EXPECT(tp_stack_plan_bytes(nullptr, 3, 3, 1) == 0);
  EXPECT(tp_stack_plan_bytes(L.data(), 0, 3, 1) == 0);
  EXPECT(tp_stack_plan_bytes(L.data(), (int)L.size(), 1, 1) == 0);
  EXPECT(tp_stack_plan_bytes(L.data(), (int)L.size(), 3, 0) == 0);
  EXPECT(tp_stack_plan_bytes(L.data(), (int)L.size(), 3, 33) == 0);
  EXPECT(tp_stack_plan_bytes(L.data(), 70000, 3, 1) == 0);
  {
    std::vector<tp_stack_linear> B = L;
    B[5].phase = 0;  // decreasing
    EXPECT(tp_stack_plan_bytes(B.data(), (int)B.size(), 3, 1) == 0);
    B = L;
    for (size_t i = 7; i < B.size(); ++i) B[i].phase += 1;  // phase 4 left empty
    EXPECT(tp_stack_plan_bytes(B.data(), (int)B.size(), 3, 1) == 0);
    B = L;
    for (auto& l : B) l.phase += 1;  // no phase 0
    EXPECT(tp_stack_plan_bytes(B.data(), (int)B.size(), 3, 1) == 0);
  }
  {
    std::vector<tp_stack_linear> B = L;
    B[2].block = 3;
    void* plan = std::aligned_alloc(256, 1 << 24);
    EXPECT(tp_stack_plan_init(B.data(), (int)B.size(), 3, 1, plan, 1 << 24) != TP_OK);
    B = L;
    B[1].x = nullptr;
    EXPECT(tp_stack_plan_init(B.data(), (int)B.size(), 3, 1, plan, 1 << 24) != TP_OK);
    B = L;
    B[1].ldy = B[1].n - 1;
    EXPECT(tp_stack_plan_init(B.data(), (int)B.size(), 3, 1, plan, 1 << 24) != TP_OK);
    EXPECT(tp_stack_plan_init(L.data(), (int)L.size(), 3, 1, static_cast<char*>(plan) + 16, 1 << 20) != TP_OK);
    std::free(plan);
  }
  int err = 0;
  EXPECT(tp_stack_error(nullptr, &err) != TP_OK);
  EXPECT(tp_stack_run(nullptr, 1, fake16(0x800000), 3, 64, 0, 1, nullptr) == TP_ERR_NULL_POINTER);
  EXPECT(tp_stack_rotate(nullptr, 1, nullptr) == TP_ERR_NULL_POINTER);
  EXPECT(tp_stack_gemv(nullptr, 1, fake16(0x800000), 3, 64, 0, 1, nullptr) == TP_ERR_NULL_POINTER);
}

static void table_and_size_cases() {
  EXPECT(tp_abi_version() > 0);
  for (int s = -64; s <= 64; ++s) EXPECT(tp_status_string(s) != nullptr);
  uint8_t lut[256];
  for (int ns : {4, 8, 16, 64}) EXPECT(tp_subset_lut(ns, lut, sizeof(lut)) == TP_OK);
  EXPECT(tp_subset_lut(32, lut, sizeof(lut)) != TP_OK);
  EXPECT(tp_subset_lut(64, lut, 64) != TP_OK);
  EXPECT(tp_subset_lut(64, nullptr, 256) != TP_OK);
  for (int64_t n : {1, 15, 16, 17, 4096, 9728})
    for (int64_t d : {1, 8, 255, 256, 257, 2560, 9728})
      for (int bits = 1; bits <= 5; ++bits) {
        int64_t t = 0, s = 0, p = 0, m = 0, z = 0;
        const int st = tp_tiled_layout(n, d, bits, &t, &s, &p, &m, &z);
        EXPECT(st == TP_OK || bits < 2 || bits > 4);
        tp_tiled_layout(n, d, bits, nullptr, nullptr, nullptr, nullptr, nullptr);
      }
  EXPECT(tp_tiled_layout(0, 256, 3, nullptr, nullptr, nullptr, nullptr, nullptr) != TP_OK);
  EXPECT(tp_tiled_layout(16, -1, 3, nullptr, nullptr, nullptr, nullptr, nullptr) != TP_OK);
  EXPECT(tp_gemv_workspace_bytes(9728, 1) >= 0);
  EXPECT(tp_gemv_workspace_bytes(9728, 32) > 0);
  EXPECT(tp_gemv_workspace_bytes(-1, 4) <= 0);
  EXPECT(tp_gemv_workspace_bytes(INT64_MAX, 32) <= 0);
  EXPECT(tp_viterbi_workspace_bytes(9728, 2560) == (int64_t)9728 * 2560 * 8);
  EXPECT(tp_viterbi_workspace_bytes(INT64_MAX, 2) <= 0);
  EXPECT(tp_viterbi_workspace_bytes(-5, 2) <= 0);
}

static void argument_cases() {
  const uint16_t* h = fake16(0x900000);
  uint16_t* o = reinterpret_cast<uint16_t*>(0xA00000);
  const uint8_t* b = fake8(0xB00000);
  EXPECT(tp_fwht_scale(nullptr, h, o, 1, 256, 256, nullptr) != TP_OK);
  EXPECT(tp_fwht_scale(h, h, o, 1, 256, 3, nullptr) != TP_OK);
  EXPECT(tp_window_decode_levels(nullptr, 4, nullptr, 0, 1, 32, 3, 64, reinterpret_cast<uint8_t*>(0xC00000), 32,
                                 nullptr) != TP_OK);
  EXPECT(tp_packed_linear_forward(nullptr, 256, 1, h, 256, b, b, h, h, nullptr, 16, 256, 3, 64, o, 16, nullptr, 0,
                                  nullptr) != TP_OK);
  EXPECT(tp_packed_linear_forward(h, 256, 0, h, 256, b, b, h, h, nullptr, 16, 256, 3, 64, o, 16, nullptr, 0,
                                  nullptr) != TP_OK);
  EXPECT(tp_packed_linear_forward(h, 256, 1, h, 256, b, b, h, h, nullptr, 16, 256, 9, 64, o, 16, nullptr, 0,
                                  nullptr) != TP_OK);
  EXPECT(tp_packed_linear_forward_noalloc(h, 256, 0, h, 256, b, b, h, h, nullptr, 16, 256, 3, 64, o, 16, nullptr) !=
         TP_OK);
  EXPECT(tp_packed_linear_forward_noalloc(h, 256, 33, h, 256, b, b, h, h, nullptr, 1 << 20, 256, 3, 64, o, 1 << 20,
                                          nullptr) == TP_ERR_BAD_DIMS);
  {
    // a split-K route (batch 6, 1024-column Hadamard blocks) one word short
    // of its workspace: refused before any launch
    const int64_t n = 33000, T = (n + 15) / 16, need = T * 16 * 16 * 4 + T * 4;
    EXPECT(tp_gemv_workspace_bytes(n, 6) >= need);
    void* ws = reinterpret_cast<void*>(0xD00000);
    EXPECT(tp_packed_linear_forward(h, 1024, 6, h, 1024, b, b, h, h, nullptr, n, 1024, 3, 64, o, n, ws, need - 4,
                                    nullptr) == TP_ERR_WORKSPACE);
  }
  EXPECT(tp_tcq_viterbi(nullptr, 256, 16, 256, nullptr, 3, 64, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                        0, nullptr) != TP_OK);
  EXPECT(tp_read_probe(nullptr, 64, nullptr, nullptr) != TP_OK);
}

int main() {
  table_and_size_cases();
  plan_cases();
  argument_cases();
  std::printf("host driver: %d unexpected results\n", failures);
  return failures ? 1 : 0;
}
