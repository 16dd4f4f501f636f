// Reference-side caller of the engine's C++ drop-in surface (the names and
// argument order of the reference's headers: include/cudalm/kernels/
// int4_gemv_bf16.h:46-52, batch_decode.h:61-79, bf16_gemv.h:19-38,
// int4_gemv.h:22-40, qwen35_kernels.h:146-155, weight_loader.h:58-63),
// compiled against include/cudalm/ and linked with libcudalm_w4a16.so. It
// is what a call site in the reference's runtime does: device buffers, the
// C++ wrappers, a stream; nothing goes through the Python layer.
//
// Usage: boundary_check DIR
// DIR/shape.txt holds "N K M". Inputs (raw little-endian): W.bin u8[N][K/2],
// S.bin fp16[N][K/128], X.bin bf16[M][K], Wg.bin/Sg.bin and Wu.bin/Su.bin
// (SwiGLU gate / up, same shapes), E.bin bf16[N][K] (tied LM head),
// Xh.bin fp16[K]. Outputs written to DIR:
//   int4_gemv_bf16.bin   bf16[N]     cudalm::int4_gemv_bf16 on row 0 of X
//   batch.bin            bf16[M][N]  cudalm::kernels::batch_int4_gemv_bf16
//   forward_host.bin     bf16[M][N]  repack_w4a16_host -> w4a16_forward_bf16
//   forward_dev.bin      bf16[M][N]  repack_w4a16 -> w4a16_forward_bf16
//   bf16_gemv.bin        bf16[N]     cudalm::bf16_gemv on row 0 of X
//   batch_bf16.bin       bf16[M][N]  cudalm::kernels::batch_bf16_gemv
//   int4_gemv.bin        fp16[N]     cudalm::int4_gemv
//   gate.bin, up.bin     bf16[M][N]  w4a16_forward_bf16 of the gate / up linears
//   silu_mul.bin         bf16[M][N]  kernels::qwen35_silu_mul_bf16(gate, up)
//   swiglu.bin           bf16[M][N]  w4a16_swiglu_forward_bf16 (one launch)
//   chain_gate.bin, chain_up.bin, chain_w.bin   bf16[M][N]  a two-stage chain
//                        over the C ABI (gate + up, then the W linear
//                        waiting for it): cudalm_w4a16_chain_plan / _run /
//                        _status
//   noalloc_w.bin        bf16[M][N]  the same chain through
//                        cudalm_w4a16_gemv_bf16_chain_noalloc
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "cudalm/kernels/batch_decode.h"
#include "cudalm/kernels/bf16_gemv.h"
#include "cudalm/kernels/int4_gemv.h"
#include "cudalm/kernels/int4_gemv_bf16.h"
#include "cudalm/kernels/swiglu.h"
#include "cudalm/w4a16_linear.h"
#include "cudalm_w4a16.h"

namespace {

std::string g_dir;

void die(const char* what) {
  std::fprintf(stderr, "boundary_check: %s\n", what);
  std::exit(2);
}

void hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "boundary_check: %s: %s\n", what, hipGetErrorString(e));
    std::exit(3);
  }
}

std::vector<std::uint8_t> read_file(const char* name, std::size_t bytes) {
  const std::string path = g_dir + "/" + name;
  std::FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) die(("cannot open " + path).c_str());
  std::vector<std::uint8_t> v(bytes);
  if (std::fread(v.data(), 1, bytes, f) != bytes) die(("short read " + path).c_str());
  std::fclose(f);
  return v;
}

void write_file(const char* name, const void* p, std::size_t bytes) {
  const std::string path = g_dir + "/" + name;
  std::FILE* f = std::fopen(path.c_str(), "wb");
  if (!f || std::fwrite(p, 1, bytes, f) != bytes) die(("cannot write " + path).c_str());
  std::fclose(f);
}

template <typename T>
T* upload(const std::vector<std::uint8_t>& h) {
  void* d = nullptr;
  hip_ok(hipMalloc(&d, h.size()), "hipMalloc");
  hip_ok(hipMemcpy(d, h.data(), h.size(), hipMemcpyHostToDevice), "upload");
  return static_cast<T*>(d);
}

template <typename T>
T* device(std::size_t bytes) {
  void* d = nullptr;
  hip_ok(hipMalloc(&d, bytes), "hipMalloc");
  hip_ok(hipMemset(d, 0xFF, bytes), "hipMemset");  // outputs must be written
  return static_cast<T*>(d);
}

void download(const char* name, const void* d, std::size_t bytes) {
  std::vector<std::uint8_t> h(bytes);
  hip_ok(hipMemcpy(h.data(), d, bytes, hipMemcpyDeviceToHost), "download");
  write_file(name, h.data(), bytes);
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 2) die("usage: boundary_check DIR");
  g_dir = argv[1];
  int N = 0, K = 0, M = 0;
  {
    const std::string path = g_dir + "/shape.txt";
    std::FILE* f = std::fopen(path.c_str(), "r");
    if (!f || std::fscanf(f, "%d %d %d", &N, &K, &M) != 3) die("bad shape.txt");
    std::fclose(f);
  }
  const std::size_t wb = static_cast<std::size_t>(N) * K / 2, sb = static_cast<std::size_t>(N) * (K / 128) * 2;
  const std::size_t xb = static_cast<std::size_t>(M) * K * 2, yb = static_cast<std::size_t>(M) * N * 2;

  hipStream_t stream;
  hip_ok(hipStreamCreate(&stream), "hipStreamCreate");

  const auto Wh = read_file("W.bin", wb);
  const auto Sh = read_file("S.bin", sb);
  auto* W = upload<std::uint8_t>(Wh);
  auto* S = upload<__half>(Sh);
  auto* X = upload<__hip_bfloat16>(read_file("X.bin", xb));
  auto* E = upload<__hip_bfloat16>(read_file("E.bin", static_cast<std::size_t>(N) * K * 2));
  auto* Xh = upload<__half>(read_file("Xh.bin", static_cast<std::size_t>(K) * 2));

  // the reference's W4A16 GEMV and batched decode entry points
  auto* y1 = device<__hip_bfloat16>(static_cast<std::size_t>(N) * 2);
  cudalm::int4_gemv_bf16(W, S, X, y1, N, K, stream);
  auto* yB = device<__hip_bfloat16>(yb);
  cudalm::kernels::batch_int4_gemv_bf16(W, S, X, yB, N, K, M, stream);
  if (cudalm::int4_gemv_bf16_rowtile4_regs() <= 0 || cudalm::kernels::batch_int4_gemv_bf16_rowtile4_regs() <= 0)
    die("register query failed");

  // load-time repack, host and device forms, then the packed forward
  std::vector<std::uint8_t> packed_h(cudalm::packed_w4a16_bytes(N, K));
  cudalm::repack_w4a16_host(Wh.data(), reinterpret_cast<const std::uint16_t*>(Sh.data()), N, K,
                            packed_h.data());
  cudalm::PackedW4A16Linear lin_h{upload<void>(packed_h), N, K};
  auto* yF = device<__hip_bfloat16>(yb);
  cudalm::w4a16_forward_bf16(lin_h, X, yF, M, stream);
  void* packed_d = device<void>(packed_h.size());
  const cudalm::PackedW4A16Linear lin_d =
      cudalm::repack_w4a16(cudalm::W4A16LinearView{W, S, N, K}, packed_d, stream);
  auto* yD = device<__hip_bfloat16>(yb);
  cudalm::w4a16_forward_bf16(lin_d, X, yD, M, stream);

  // the tied bf16 LM head and the fp16-activation twin
  auto* yE = device<__hip_bfloat16>(static_cast<std::size_t>(N) * 2);
  cudalm::bf16_gemv(E, X, yE, N, K, stream);
  auto* yEB = device<__hip_bfloat16>(yb);
  cudalm::kernels::batch_bf16_gemv(E, X, yEB, N, K, M, stream);
  auto* yH = device<__half>(static_cast<std::size_t>(N) * 2);
  cudalm::int4_gemv(W, S, Xh, yH, N, K, stream);

  // MLP front half: gate and up, silu*mul, and the fused launch
  auto* Wg = upload<std::uint8_t>(read_file("Wg.bin", wb));
  auto* Sg = upload<__half>(read_file("Sg.bin", sb));
  auto* Wu = upload<std::uint8_t>(read_file("Wu.bin", wb));
  auto* Su = upload<__half>(read_file("Su.bin", sb));
  const cudalm::PackedW4A16Linear gate = cudalm::repack_w4a16(
      cudalm::W4A16LinearView{Wg, Sg, N, K}, device<void>(packed_h.size()), stream);
  const cudalm::PackedW4A16Linear up = cudalm::repack_w4a16(
      cudalm::W4A16LinearView{Wu, Su, N, K}, device<void>(packed_h.size()), stream);
  auto* yg = device<__hip_bfloat16>(yb);
  auto* yu = device<__hip_bfloat16>(yb);
  auto* ysm = device<__hip_bfloat16>(yb);
  auto* ysw = device<__hip_bfloat16>(yb);
  cudalm::w4a16_forward_bf16(gate, X, yg, M, stream);
  cudalm::w4a16_forward_bf16(up, X, yu, M, stream);
  cudalm::kernels::qwen35_silu_mul_bf16(yg, yu, ysm, static_cast<std::size_t>(M) * N, stream);
  cudalm::w4a16_swiglu_forward_bf16(gate, up, X, ysw, M, stream);

  // stage chains (C ABI): gate and up as one stage, then the W linear
  // waiting for it; then the same stages without a workspace
  auto* ycg = device<std::uint16_t>(yb);
  auto* ycu = device<std::uint16_t>(yb);
  auto* ycw = device<std::uint16_t>(yb);
  auto* ycn = device<std::uint16_t>(yb);
  {
    const auto* xs = reinterpret_cast<const std::uint16_t*>(X);
    const cudalm_w4a16_proj gu[2] = {{gate.packed, nullptr, ycg, N}, {up.packed, nullptr, ycu, N}};
    const cudalm_w4a16_proj lw[1] = {{lin_d.packed, nullptr, ycw, N}};
    const cudalm_w4a16_proj ln[1] = {{lin_d.packed, nullptr, ycn, N}};
    const cudalm_w4a16_stage stages[2] = {{gu, 2, xs, K, -1}, {lw, 1, xs, K, 0}};
    const cudalm_w4a16_stage stages_n[2] = {{gu, 2, xs, K, -1}, {ln, 1, xs, K, 0}};
    const std::size_t wsb = cudalm_w4a16_chain_workspace_bytes(2);
    void* ws = device<void>(wsb);
    cudalm_w4a16_chain chain;
    if (cudalm_w4a16_chain_plan(stages, 2, M, 1, ws, wsb, &chain, stream) != 0) die("chain plan");
    if (cudalm_w4a16_chain_run(&chain, stream) != 0) die("chain run");
    if (cudalm_w4a16_chain_status(&chain, stream) != 0) die("chain status");
    if (cudalm_w4a16_gemv_bf16_chain_noalloc(stages_n, 2, M, 1, stream) != 0) die("chain noalloc");
  }

  hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize");
  download("chain_gate.bin", ycg, yb);
  download("chain_up.bin", ycu, yb);
  download("chain_w.bin", ycw, yb);
  download("noalloc_w.bin", ycn, yb);
  download("int4_gemv_bf16.bin", y1, static_cast<std::size_t>(N) * 2);
  download("batch.bin", yB, yb);
  download("forward_host.bin", yF, yb);
  download("forward_dev.bin", yD, yb);
  download("bf16_gemv.bin", yE, static_cast<std::size_t>(N) * 2);
  download("batch_bf16.bin", yEB, yb);
  download("int4_gemv.bin", yH, static_cast<std::size_t>(N) * 2);
  download("gate.bin", yg, yb);
  download("up.bin", yu, yb);
  download("silu_mul.bin", ysm, yb);
  download("swiglu.bin", ysw, yb);
  std::printf("boundary_check: N=%d K=%d M=%d ok\n", N, K, M);
  return 0;
}
