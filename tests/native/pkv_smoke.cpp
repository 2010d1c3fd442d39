// pkv_smoke.cpp — native smoke test of the engine through its C ABI (include/pkv.h), with
// no Python and no torch: the counterpart of the reference's tests/smoke_test.cu.
//
// For each of the reference's eight correctness cases (smoke_test.cu:486-493) it draws the
// inputs the reference draws (glibc srand(42)/rand(), quantised to fp16, :77-81, :125-138),
// runs them through libpkv.so, and checks the output against the fp32 CPU attention of
// smoke_test.cu:35-74 with the reference's gate, max-abs < 2e-3 and mean-abs < 3e-4
// (:106, :205).  Contiguous cases go through pkv_attention_contiguous (the reference runs
// them through persistentkv_dispatch / persistentkv_split_dispatch, :155-163), case 0 also
// through pkv_attention_query_head_baseline (:176-192); paged cases store the pages in
// reversed physical order behind a block table (:239-258) and go through
// pkv_paged_attention.
//
// The inputs and the CPU attention come from the test oracle (oracle/pkv_oracle.c,
// libpkv_oracle.so), the checker; the engine under test is libpkv.so.
// Exit status: 0 when every case passes, 1 when one fails the gate, 2 on an API error.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "pkv.h"

extern "C" {
int pkv_oracle_smoke_case(int index, int* shape6);
int pkv_oracle_smoke_inputs(int index, float* q, float* k, float* v);
void pkv_oracle_cpu_gqa_attention(const float* Q, const float* K, const float* V, float* O,
                                  int B, int Hq, int Hkv, int N, int d);
}

namespace {

constexpr int kD = PKV_HEAD_DIM;
constexpr double kMaxAbs = 2e-3, kMeanAbs = 3e-4;

[[noreturn]] void die(const char* what, const char* detail) {
  std::fprintf(stderr, "pkv_smoke: %s: %s\n", what, detail);
  std::exit(2);
}

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) die(what, hipGetErrorString(e));
}

void pkv_check(int status, const char* what) {
  if (status != PKV_OK) die(what, pkv_last_error());
}

// Device buffer of `n` elements of T, freed on scope exit.
template <class T>
struct DeviceBuffer {
  T* ptr = nullptr;
  size_t n = 0;
  explicit DeviceBuffer(size_t count) : n(count) {
    hip_check(hipMalloc((void**)&ptr, (count ? count : 1) * sizeof(T)), "hipMalloc");
  }
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  ~DeviceBuffer() { (void)hipFree(ptr); }
  void upload(const std::vector<T>& h) {
    hip_check(hipMemcpy(ptr, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice), "upload");
  }
  std::vector<T> download() const {
    std::vector<T> h(n);
    hip_check(hipMemcpy(h.data(), ptr, n * sizeof(T), hipMemcpyDeviceToHost), "download");
    return h;
  }
};

struct Error {
  double max_abs = 0, mean_abs = 0;
  bool pass() const { return max_abs < kMaxAbs && mean_abs < kMeanAbs; }
};

Error compare(const std::vector<_Float16>& got, const std::vector<float>& want) {
  Error e;
  double sum = 0;
  for (size_t i = 0; i < want.size(); ++i) {
    const double d = std::fabs((double)(float)got[i] - (double)want[i]);
    if (!(d <= e.max_abs)) e.max_abs = std::isnan(d) ? INFINITY : d;
    sum += d;
  }
  e.mean_abs = want.empty() ? 0 : sum / (double)want.size();
  return e;
}

bool report(int index, const char* path, const int* s, const Error& e) {
  std::printf("case %d %-10s B=%d Hq=%d Hkv=%d N=%d S=%d page=%d  max_abs=%.3e mean_abs=%.3e  %s\n",
              index, path, s[0], s[1], s[2], s[3], s[4], s[5], e.max_abs, e.mean_abs,
              e.pass() ? "PASS" : "FAIL");
  std::fflush(stdout);
  return e.pass();
}

bool run_case(int index, hipStream_t stream) {
  int s[6];
  if (pkv_oracle_smoke_case(index, s) != 0) die("smoke case", "index out of range");
  const int B = s[0], Hq = s[1], Hkv = s[2], N = s[3], S = s[4], ps = s[5];
  const size_t qn = (size_t)B * Hq * kD, kvn = (size_t)B * Hkv * N * kD;

  // Inputs as the reference draws them, quantised to fp16; the CPU attention sees the
  // quantised values.
  std::vector<float> qf(qn), kf(kvn), vf(kvn);
  pkv_oracle_smoke_inputs(index, qf.data(), kf.data(), vf.data());
  std::vector<_Float16> qh(qn), kh(kvn), vh(kvn);
  for (size_t i = 0; i < qn; ++i) qf[i] = (float)(qh[i] = (_Float16)qf[i]);
  for (size_t i = 0; i < kvn; ++i) kf[i] = (float)(kh[i] = (_Float16)kf[i]);
  for (size_t i = 0; i < kvn; ++i) vf[i] = (float)(vh[i] = (_Float16)vf[i]);
  std::vector<float> ref(qn);
  pkv_oracle_cpu_gqa_attention(qf.data(), kf.data(), vf.data(), ref.data(), B, Hq, Hkv, N, kD);

  DeviceBuffer<_Float16> q(qn), out(qn);
  q.upload(qh);
  DeviceBuffer<float> ws(pkv_workspace_bytes(B, Hq, S) / sizeof(float));
  const size_t ws_bytes = ws.n * sizeof(float);
  bool ok = true;

  if (ps == 0) {
    DeviceBuffer<_Float16> k(kvn), v(kvn);
    k.upload(kh);
    v.upload(vh);
    pkv_check(pkv_attention_contiguous(q.ptr, k.ptr, v.ptr, out.ptr, ws.ptr, ws_bytes, B, Hq, Hkv,
                                       N, kD, S, PKV_DTYPE_F16, stream),
              "pkv_attention_contiguous");
    hip_check(hipStreamSynchronize(stream), "contiguous");
    ok &= report(index, "contiguous", s, compare(out.download(), ref));
    if (index == 0) {
      pkv_check(pkv_attention_query_head_baseline(q.ptr, k.ptr, v.ptr, out.ptr, B, Hq, Hkv, N, kD,
                                                  PKV_DTYPE_F16, stream),
                "pkv_attention_query_head_baseline");
      hip_check(hipStreamSynchronize(stream), "baseline");
      ok &= report(index, "baseline", s, compare(out.download(), ref));
    }
    return ok;
  }

  // Paged: row b's logical page p lives in physical page b*ppb + (ppb - 1 - p).
  const int ppb = (N + ps - 1) / ps, pages = B * ppb;
  std::vector<_Float16> kp((size_t)pages * Hkv * ps * kD, (_Float16)0.f), vp(kp.size(), (_Float16)0.f);
  std::vector<int32_t> table((size_t)B * ppb);
  for (int b = 0; b < B; ++b)
    for (int p = 0; p < ppb; ++p) {
      const int phys = b * ppb + (ppb - 1 - p);
      table[(size_t)b * ppb + p] = phys;
      for (int h = 0; h < Hkv; ++h)
        for (int t = p * ps; t < N && t < (p + 1) * ps; ++t)
          for (int d = 0; d < kD; ++d) {
            const size_t src = (((size_t)b * Hkv + h) * N + t) * kD + d;
            const size_t dst = (((size_t)phys * Hkv + h) * ps + (t - p * ps)) * kD + d;
            kp[dst] = kh[src];
            vp[dst] = vh[src];
          }
    }
  DeviceBuffer<_Float16> k(kp.size()), v(vp.size());
  DeviceBuffer<int32_t> bt(table.size());
  k.upload(kp);
  v.upload(vp);
  bt.upload(table);
  pkv_check(pkv_paged_attention(q.ptr, k.ptr, v.ptr, bt.ptr, out.ptr, ws.ptr, ws_bytes, B, Hq, Hkv,
                                kD, pages, ps, ppb, N, S, PKV_DTYPE_F16, stream),
            "pkv_paged_attention");
  hip_check(hipStreamSynchronize(stream), "paged");
  return report(index, "paged", s, compare(out.download(), ref));
}

}  // namespace

int main() {
  int devices = 0;
  hip_check(hipGetDeviceCount(&devices), "hipGetDeviceCount");
  if (devices < 1) die("hipGetDeviceCount", "no GPU");
  hip_check(hipSetDevice(0), "hipSetDevice");
  hipStream_t stream;
  hip_check(hipStreamCreate(&stream), "hipStreamCreate");
  std::printf("pkv_smoke: libpkv version %d, reference smoke cases (fp16, gate max_abs < %.0e, "
              "mean_abs < %.0e)\n", pkv_version(), kMaxAbs, kMeanAbs);
  bool ok = true;
  for (int i = 0; i < 8; ++i) ok &= run_case(i, stream);
  hip_check(hipStreamDestroy(stream), "hipStreamDestroy");
  std::printf("pkv_smoke: %s\n", ok ? "all cases passed" : "FAILED");
  return ok ? 0 : 1;
}
