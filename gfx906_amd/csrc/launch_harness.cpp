// A torch-free C caller of the attention library's launch() entry point, in
// the manner of the reference's micro3.hip (micro3.hip:4-17: hipMalloc the
// buffers, call launch(...) on stream 0, time it with hipEvents). It links
// against libgfx906_amd_attn.so like any C/C++ program that uses the C ABI
// (include/gfx906_amd_attn.h) and needs neither Python nor PyTorch.
//
// usage: launch_harness DIR B H Sq Skv D SCALE REPS
//   reads DIR/q.bin ([B,H,Sq,D] fp16), DIR/k.bin and DIR/v.bin ([B,H,Skv,D]
//   fp16), runs launch() once, writes the output to DIR/o.bin, then times
//   REPS further launches back to back and prints one JSON line:
//   {"ms_avg": ..., "ms_min": ..., "tflops": ...}.
// Exit status: 0 on success, 1 for bad usage or I/O, 2 for a HIP or library
// error (message on stderr).
#include <hip/hip_runtime.h>

#include <stdio.h>
#include <stdlib.h>
#include <string>
#include <vector>

#include "gfx906_amd_attn.h"

namespace {

bool read_file(const std::string& path, std::vector<unsigned char>& buf, size_t bytes) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return false;
    buf.resize(bytes);
    const size_t got = bytes ? fread(buf.data(), 1, bytes, f) : 0;
    const bool extra = fgetc(f) != EOF;
    fclose(f);
    return got == bytes && !extra;
}

bool write_file(const std::string& path, const std::vector<unsigned char>& buf) {
    FILE* f = fopen(path.c_str(), "wb");
    if (!f) return false;
    const size_t put = buf.empty() ? 0 : fwrite(buf.data(), 1, buf.size(), f);
    return fclose(f) == 0 && put == buf.size();
}

int hip_fail(const char* what, hipError_t e) {
    fprintf(stderr, "launch_harness: %s: %s\n", what, hipGetErrorString(e));
    return 2;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 9) {
        fprintf(stderr, "usage: %s DIR B H Sq Skv D SCALE REPS\n", argv[0]);
        return 1;
    }
    const std::string dir = argv[1];
    const int B = atoi(argv[2]), H = atoi(argv[3]), Sq = atoi(argv[4]), Skv = atoi(argv[5]),
              D = atoi(argv[6]);
    const float scale = (float)atof(argv[7]);
    const int reps = atoi(argv[8]);
    if (B <= 0 || H <= 0 || Sq <= 0 || Skv < 0 || D <= 0 || reps < 0) {
        fprintf(stderr, "launch_harness: bad sizes\n");
        return 1;
    }
    const size_t nq = (size_t)B * H * Sq * D * 2, nk = (size_t)B * H * Skv * D * 2;
    std::vector<unsigned char> hq, hk, hv;
    if (!read_file(dir + "/q.bin", hq, nq) || !read_file(dir + "/k.bin", hk, nk) ||
        !read_file(dir + "/v.bin", hv, nk)) {
        fprintf(stderr, "launch_harness: cannot read %s/{q,k,v}.bin of the given sizes\n",
                dir.c_str());
        return 1;
    }
    void *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
    hipError_t e;
    if ((e = hipMalloc(&q, nq)) != hipSuccess || (e = hipMalloc(&k, nk ? nk : 16)) != hipSuccess ||
        (e = hipMalloc(&v, nk ? nk : 16)) != hipSuccess || (e = hipMalloc(&o, nq)) != hipSuccess)
        return hip_fail("hipMalloc", e);
    if ((e = hipMemcpy(q, hq.data(), nq, hipMemcpyHostToDevice)) != hipSuccess ||
        (nk && (e = hipMemcpy(k, hk.data(), nk, hipMemcpyHostToDevice)) != hipSuccess) ||
        (nk && (e = hipMemcpy(v, hv.data(), nk, hipMemcpyHostToDevice)) != hipSuccess))
        return hip_fail("hipMemcpy to device", e);

    launch(q, k, v, o, B, H, Sq, Skv, D, scale, 0);
    if (const char* err = attn_last_error()) {
        fprintf(stderr, "launch_harness: launch: %s\n", err);
        return 2;
    }
    if ((e = hipDeviceSynchronize()) != hipSuccess) return hip_fail("first launch", e);
    std::vector<unsigned char> ho(nq);
    if ((e = hipMemcpy(ho.data(), o, nq, hipMemcpyDeviceToHost)) != hipSuccess)
        return hip_fail("hipMemcpy to host", e);
    if (!write_file(dir + "/o.bin", ho)) {
        fprintf(stderr, "launch_harness: cannot write %s/o.bin\n", dir.c_str());
        return 1;
    }

    double sum = 0.0, best = 0.0;
    if (reps > 0) {
        hipEvent_t a, b;
        if ((e = hipEventCreate(&a)) != hipSuccess || (e = hipEventCreate(&b)) != hipSuccess)
            return hip_fail("hipEventCreate", e);
        for (int r = 0; r < reps; ++r) {
            hipEventRecord(a, 0);
            launch(q, k, v, o, B, H, Sq, Skv, D, scale, 0);
            hipEventRecord(b, 0);
            if ((e = hipEventSynchronize(b)) != hipSuccess) return hip_fail("timed launch", e);
            float ms = 0.f;
            hipEventElapsedTime(&ms, a, b);
            sum += ms;
            best = r == 0 || ms < best ? ms : best;
        }
        hipEventDestroy(a);
        hipEventDestroy(b);
    }
    const double avg = reps > 0 ? sum / reps : 0.0;
    const double flops = 4.0 * B * H * (double)Sq * Skv * D;
    printf("{\"ms_avg\": %.5f, \"ms_min\": %.5f, \"tflops\": %.2f}\n", avg, best,
           avg > 0 ? flops / (avg * 1e-3) / 1e12 : 0.0);
    hipFree(q);
    hipFree(k);
    hipFree(v);
    hipFree(o);
    return 0;
}
