// One wave records the lane semantics of the gfx950 instructions the emulation
// models (tests/emu/include/hip/hip_runtime.h): the transposing LDS read, the two
// bf16 MFMA shapes, v_permlane32_swap and the DPP controls of the library's
// reductions.  Built with hipcc and run on an MI355X it wrote
// fixtures/gfx950_lanes.bin; built through the emulation it must write the same.
//
//     hipcc --offload-arch=gfx950 -O2 -o probe_lanes probe_lanes.hip && ./probe_lanes out.bin
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
typedef __attribute__((address_space(3))) char lds_char_t;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int NOUT = 1920 + 64 * 8;

__global__ __launch_bounds__(64) void probe(const uint16_t* a32, const uint16_t* b32, const uint16_t* a16,
                                            const uint16_t* b16, uint32_t* out) {
  __shared__ uint16_t lds[64 * 16];
  const int l = threadIdx.x;
  for (int i = l; i < 64 * 16; i += 64) lds[i] = (uint16_t)i;
  __syncthreads();
  // the transposing read, lane address 8 l bytes, then (l % 16) 32 + (l / 16) 8 bytes
  s16x4_t t = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)((lds_char_t*)lds + l * 8));
  for (int e = 0; e < 4; ++e) out[l * 4 + e] = (uint16_t)t[e];
  s16x4_t t2 =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)((lds_char_t*)lds + (l % 16) * 32 + (l / 16) * 8));
  for (int e = 0; e < 4; ++e) out[256 + l * 4 + e] = (uint16_t)t2[e];
  // mfma 32x32x16 and 16x16x32 bf16 of the given operands
  bf16x8_t av, bv;
  memcpy(&av, a32 + l * 8, 16);
  memcpy(&bv, b32 + l * 8, 16);
  f32x16_t c = {};
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, c, 0, 0, 0);
  for (int e = 0; e < 16; ++e) out[512 + l * 16 + e] = __float_as_uint(c[e]);
  bf16x8_t a2, b2;
  memcpy(&a2, a16 + l * 8, 16);
  memcpy(&b2, b16 + l * 8, 16);
  f32x4_t c2 = {};
  c2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b2, c2, 0, 0, 0);
  for (int e = 0; e < 4; ++e) out[1536 + l * 4 + e] = __float_as_uint(c2[e]);
  // permlane32_swap(lane, 100 + lane)
  auto r = __builtin_amdgcn_permlane32_swap((uint32_t)l, (uint32_t)(100 + l), false, false);
  out[1792 + l * 2] = r[0];
  out[1792 + l * 2 + 1] = r[1];
  // update_dpp (old 0, bound_ctrl) with the library's controls
  const int v = 1000 + l;
  out[1920 + l * 8 + 0] = __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, true);
  out[1920 + l * 8 + 1] = __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, true);
  out[1920 + l * 8 + 2] = __builtin_amdgcn_update_dpp(0, v, 0x124, 0xf, 0xf, true);
  out[1920 + l * 8 + 3] = __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, true);
  out[1920 + l * 8 + 4] = __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);
  out[1920 + l * 8 + 5] = __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);
  out[1920 + l * 8 + 6] = __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);
  out[1920 + l * 8 + 7] = __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);
}

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  std::vector<uint16_t> a32(512), b32(512), a16(512), b16(512);
  uint32_t s = 12345;
  auto rnd = [&]() {
    s = s * 1103515245u + 12345u;
    return (int)((s >> 16) % 7) - 3;
  };
  auto bf = [](float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)(u >> 16);
  };
  for (int i = 0; i < 512; ++i) {
    a32[i] = bf((float)rnd());
    b32[i] = bf((float)rnd());
    a16[i] = bf((float)rnd());
    b16[i] = bf((float)rnd());
  }
  uint16_t *da32, *db32, *da16, *db16;
  uint32_t* dout;
  if (hipMalloc(&da32, 1024) || hipMalloc(&db32, 1024) || hipMalloc(&da16, 1024) || hipMalloc(&db16, 1024) ||
      hipMalloc(&dout, NOUT * 4))
    return 1;
  hipMemcpy(da32, a32.data(), 1024, hipMemcpyHostToDevice);
  hipMemcpy(db32, b32.data(), 1024, hipMemcpyHostToDevice);
  hipMemcpy(da16, a16.data(), 1024, hipMemcpyHostToDevice);
  hipMemcpy(db16, b16.data(), 1024, hipMemcpyHostToDevice);
  hipMemset(dout, 0, NOUT * 4);
  hipLaunchKernelGGL(probe, dim3(1), dim3(64), 0, 0, da32, db32, da16, db16, dout);
  std::vector<uint32_t> out(NOUT);
  hipMemcpy(out.data(), dout, NOUT * 4, hipMemcpyDeviceToHost);
  if (hipDeviceSynchronize() != hipSuccess) return 1;
  FILE* f = fopen(argv[1], "wb");
  if (!f) return 1;
  fwrite(a32.data(), 2, 512, f);
  fwrite(b32.data(), 2, 512, f);
  fwrite(a16.data(), 2, 512, f);
  fwrite(b16.data(), 2, 512, f);
  fwrite(out.data(), 4, NOUT, f);
  fclose(f);
  return 0;
}
