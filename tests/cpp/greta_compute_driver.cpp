// Drives the C++ host mirror end to end, as a caller of the reference's
// interfaces would: create_weight_loader -> GGUFLoader::load_tensor_quant /
// load_tensor_int8 / load_tensor_int4 (or, for a .greta file, GretaLoader's
// load_tensor_quant / load_tensor_int4) -> GretaCompute::gemm on a
// GretaStreamHip.  Test infrastructure: tests/test_host_mirror.py runs it and
// checks the result file against the oracle.
//
// usage: greta_compute_driver <file.gguf|file.greta> <tensor> <quant|int8|int4|fp16> <M>
//                             <a.f32> <c.f32> [op_label] [a_dtype f32|f16|bf16]
// A is read as M x K float32 (converted to the requested A dtype on the host),
// C written as M x N float32.  Prints "route=<GEMV|GEMM|VALU|MFMA> quant=<mode>".
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iostream>
#include <string>
#include <vector>

#include "gcore/compute/greta_compute.hpp"
#include "gcore/inference/greta_file.hpp"
#include "gcore/inference/weight_loader.hpp"
#include "gcore/rt/hip/buffer.hpp"
#include "gcore/rt/hip/greta_runtime_hip.hpp"

using namespace gcore;

static uint16_t f32_to_f16_rne(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
static uint16_t f32_to_bf16_rne(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  x += 0x7FFFu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

static int fail(const std::string &m) {
  std::cerr << "greta_compute_driver: " << m << std::endl;
  return 1;
}

int main(int argc, char **argv) {
  if (argc < 7) return fail("usage: file.gguf tensor quant|int8|int4 M a.f32 c.f32 [label] [a_dtype]");
  const std::string path = argv[1], name = argv[2], kind = argv[3];
  const uint32_t M = (uint32_t)std::stoul(argv[4]);
  const std::string label = argc > 7 ? argv[7] : "";
  const std::string adt = argc > 8 ? argv[8] : "f32";
  std::string err;

  auto wl = inference::create_weight_loader(path, &err);
  if (!wl) return fail("open: " + err);
  auto *gg = dynamic_cast<inference::GGUFLoader *>(wl.get());
  auto *gr = dynamic_cast<inference::GretaLoader *>(wl.get());
  if (!gg && !gr) return fail("neither a GGUF nor a .greta loader");
  size_t K = 0, n_elem = 1;
  for (const auto &t : wl->list_tensors())
    if (t.name == name) {
      K = t.shape[0];
      for (size_t d : t.shape) n_elem *= d;
    }
  if (K == 0) return fail("tensor not found: " + name);
  const uint32_t N = (uint32_t)(n_elem / K);

  rt::hip::Buffer B, scales, head_scales;
  bool ok = kind == "quant"  ? (gg ? gg->load_tensor_quant(name, B, &err) : gr->load_tensor_quant(name, B, &err))
            : kind == "int8" ? wl->load_tensor_int8(name, B, scales, &err)
            : kind == "int4" ? wl->load_tensor_int4(name, B, scales, head_scales, &err)
            : kind == "fp16" ? wl->load_tensor_fp16(name, B, &err)
                             : (err = "unknown kind " + kind, false);
  if (!ok) return fail("load: " + err);

  std::vector<float> a((size_t)M * K);
  {
    std::ifstream f(argv[5], std::ios::binary);
    if (!f.read(reinterpret_cast<char *>(a.data()), a.size() * 4)) return fail("cannot read A");
  }
  rt::hip::Buffer A, C;
  if (adt == "f32") {
    if (!A.allocate(a.size() * 4, rt::hip::BufferUsage::DeviceOnly, rt::GretaDataType::FP32, &err) ||
        !A.copy_to_device(a.data(), a.size() * 4, &err))
      return fail("A: " + err);
  } else {
    std::vector<uint16_t> h(a.size());
    for (size_t i = 0; i < a.size(); ++i) h[i] = adt == "f16" ? f32_to_f16_rne(a[i]) : f32_to_bf16_rne(a[i]);
    auto t = adt == "f16" ? rt::GretaDataType::FP16 : rt::GretaDataType::BF16;
    if (!A.allocate(h.size() * 2, rt::hip::BufferUsage::DeviceOnly, t, &err) ||
        !A.copy_to_device(h.data(), h.size() * 2, &err))
      return fail("A: " + err);
  }
  if (!C.allocate((size_t)M * N * 4, rt::hip::BufferUsage::DeviceOnly, rt::GretaDataType::FP32, &err))
    return fail("C: " + err);

  rt::hip::GretaStreamHip stream;
  compute::GretaCompute::set_op_label(label.c_str());
  rt::GretaResult r = compute::GretaCompute::gemm(&stream, &A, &B, &C, M, N, (uint32_t)K);
  stream.synchronize();
  if (r != rt::GretaResult::SUCCESS) return fail("gemm returned " + std::to_string((int)r));
  std::vector<float> c((size_t)M * N);
  if (!C.copy_to_host(c.data(), c.size() * 4, &err)) return fail("C copy: " + err);
  std::ofstream o(argv[6], std::ios::binary);
  o.write(reinterpret_cast<const char *>(c.data()), c.size() * 4);
  auto au = compute::GretaCompute::get_last_gemm_audit();
  std::cout << "route=" << au.route << " quant=" << au.quant_mode << " N=" << N << " K=" << K << std::endl;
  return 0;
}
