// Host-side sanitizer check of the C-ABI library (test infrastructure).
//
// Built by tests/test_sanitizers.py with AddressSanitizer and
// UndefinedBehaviorSanitizer on the host code of every library source (the
// device code is unchanged), and run on a machine without a GPU.  Every
// entry point is called from a small valid configuration with one argument
// at a time replaced by an extreme value (negative, zero, 2^31, 2^62,
// INT64_MAX, ...) or one pointer set to NULL.  Without a device, a call
// that passes validation fails at its first HIP call, so no kernel ever
// runs; the tensor pointers are unmapped addresses, so any host-side read
// of device memory faults.  What is checked: no sanitizer report (the
// sanitizers abort the process), every status is one of the DSA_* codes,
// NULL tensors are rejected with DSA_ERR_INVALID, and every non-OK status
// leaves a message in dsa_last_error().
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <functional>
#include <string>
#include <thread>
#include <vector>

#include "dsa_capi.h"

namespace {

typedef std::vector<int64_t> Ints;
typedef std::vector<const void*> Ptrs;

const int64_t kExtremes[] = {-1, 0, 1, 3, 65, 4097, (1ll << 31) - 1, 1ll << 31, 1ll << 40, 1ll << 62,
                             INT64_MAX, INT64_MIN};

int g_cases = 0, g_fail = 0;

void fail(const std::string& what) {
  ++g_fail;
  fprintf(stderr, "FAIL %s\n", what.c_str());
}

struct Entry {
  const char* name;
  Ints ints;                                  // every integer argument, in order
  int nptr;                                   // tensor pointer arguments
  std::vector<int> optional;                  // pointers that may be NULL
  std::function<int(const Ptrs&, const Ints&)> call;
};

const void* P(const Ptrs& p, int i) { return p[i]; }
int32_t I32(const Ints& v, int i) { return (int32_t)v[i]; }

void run_case(const Entry& e, const Ptrs& p, const Ints& v, const std::string& label, bool must_reject_null) {
  ++g_cases;
  const int st = e.call(p, v);
  if (st < DSA_OK || st > DSA_ERR_WORKSPACE) fail(label + ": status " + std::to_string(st));
  if (st != DSA_OK && dsa_last_error()[0] == '\0') fail(label + ": empty error message");
  if (must_reject_null && st != DSA_ERR_INVALID) fail(label + ": NULL tensor not rejected (" + std::to_string(st) + ")");
}

void sweep(const Entry& e) {
  Ptrs base;
  for (int i = 0; i < e.nptr; ++i) base.push_back((const void*)(uintptr_t)(0x10000 + 0x1000 * i));
  run_case(e, base, e.ints, std::string(e.name) + " baseline", false);
  for (size_t i = 0; i < e.ints.size(); ++i) {
    for (int64_t x : kExtremes) {
      Ints v = e.ints;
      v[i] = x;
      run_case(e, base, v, std::string(e.name) + " int arg " + std::to_string(i) + " = " + std::to_string(x), false);
    }
  }
  for (int i = 0; i < e.nptr; ++i) {
    Ptrs p = base;
    p[i] = nullptr;
    bool opt = false;
    for (int o : e.optional) opt |= (o == i);
    run_case(e, p, e.ints, std::string(e.name) + " ptr " + std::to_string(i) + " = NULL", !opt);
  }
}

void sweep_size(const char* name, Ints ints, const std::function<size_t(const Ints&)>& fn) {
  for (size_t i = 0; i < ints.size(); ++i)
    for (int64_t x : kExtremes) {
      Ints v = ints;
      v[i] = x;
      ++g_cases;
      (void)fn(v);
    }
  (void)name;
}

const int64_t kMax = INT64_MAX;

}  // namespace

int main() {
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) == hipSuccess && ndev > 0) {
    // calls that pass validation would launch kernels on dummy pointers
    printf("SKIP a GPU is present\n");
    return 0;
  }
  std::vector<Entry> entries;
  // dsa_sfa_fwd: 11 tensors (softmax_max/sum, act lengths and block_table optional)
  entries.push_back({"dsa_sfa_fwd",
                     {1, 4, 256, 8, 128, 64, 64, 4, 256, 0, 0, 1, 0, kMax, kMax, 0, 0, 0, 1, 1ll << 30},
                     11, {6, 7, 8, 9, 10},
                     [](const Ptrs& p, const Ints& v) {
                       return dsa_sfa_fwd(P(p, 0), P(p, 1), P(p, 2), P(p, 3), (const int32_t*)P(p, 4), (void*)P(p, 5),
                                          (float*)P(p, 6), (float*)P(p, 7), (const int32_t*)P(p, 8),
                                          (const int32_t*)P(p, 9), (const int32_t*)P(p, 10), v[0], v[1], v[2], v[3],
                                          v[4], v[5], v[6], v[7], v[8], v[9], v[10], I32(v, 11), I32(v, 12), v[13],
                                          v[14], I32(v, 15), I32(v, 16), I32(v, 17), 0.1f, I32(v, 18),
                                          (void*)0x7f0000, (size_t)v[19], nullptr);
                     }});
  entries.push_back({"dsa_sfa_fwd_noalloc",
                     {1, 4, 256, 8, 128, 64, 64, 4, 256, 0, 0, 1, 0, kMax, kMax, 0, 0, 0, 1},
                     11, {6, 7, 8, 9, 10},
                     [](const Ptrs& p, const Ints& v) {
                       return dsa_sfa_fwd_noalloc(P(p, 0), P(p, 1), P(p, 2), P(p, 3), (const int32_t*)P(p, 4),
                                                  (void*)P(p, 5), (float*)P(p, 6), (float*)P(p, 7),
                                                  (const int32_t*)P(p, 8), (const int32_t*)P(p, 9),
                                                  (const int32_t*)P(p, 10), v[0], v[1], v[2], v[3], v[4], v[5], v[6],
                                                  v[7], v[8], v[9], v[10], I32(v, 11), I32(v, 12), v[13], v[14],
                                                  I32(v, 15), I32(v, 16), I32(v, 17), 0.1f, I32(v, 18), nullptr);
                     }});
  // dsa_sfa_bwd: 16 tensors (act lengths and d_value optional)
  entries.push_back({"dsa_sfa_bwd",
                     {1, 4, 256, 8, 128, 64, 64, 4, 256, 1, 3, kMax, kMax, 0, 0, 1ll << 34},
                     16, {9, 10, 15},
                     [](const Ptrs& p, const Ints& v) {
                       return dsa_sfa_bwd(P(p, 0), P(p, 1), P(p, 2), P(p, 3), (const int32_t*)P(p, 4), P(p, 5), P(p, 6),
                                          (const float*)P(p, 7), (const float*)P(p, 8), (const int32_t*)P(p, 9),
                                          (const int32_t*)P(p, 10), (void*)P(p, 11), (void*)P(p, 12), (void*)P(p, 13),
                                          (void*)P(p, 14), (void*)P(p, 15), v[0], v[1], v[2], v[3], v[4], v[5], v[6],
                                          v[7], v[8], I32(v, 9), I32(v, 10), v[11], v[12], I32(v, 13), I32(v, 14),
                                          0.1f, (void*)0x7f0000, (size_t)v[15], nullptr);
                     }});
  // dsa_kl_bwd: 16 tensors (rope and act lengths optional)
  entries.push_back({"dsa_kl_bwd",
                     {1, 16, 16, 8, 128, 64, 8, 128, 16, 0, 2, 1ll << 30},
                     16, {2, 3, 10, 11},
                     [](const Ptrs& p, const Ints& v) {
                       return dsa_kl_bwd(P(p, 0), P(p, 1), P(p, 2), P(p, 3), P(p, 4), P(p, 5), P(p, 6),
                                         (const int32_t*)P(p, 7), (const float*)P(p, 8), (const float*)P(p, 9),
                                         (const int32_t*)P(p, 10), (const int32_t*)P(p, 11), (void*)P(p, 12),
                                         (void*)P(p, 13), (void*)P(p, 14), (float*)P(p, 15), v[0], v[1], v[2], v[3],
                                         v[4], v[5], v[6], v[7], v[8], I32(v, 9), I32(v, 10), 0.1f, (void*)0x7f0000,
                                         (size_t)v[11], nullptr);
                     }});
  entries.push_back({"dsa_kl_bwd_ex",
                     {1, 16, 16, 8, 128, 64, 8, 128, 16, 16, 16, 0, 0, 0, 0, 0, 2, 1ll << 30},
                     17, {2, 3, 10, 11, 12},
                     [](const Ptrs& p, const Ints& v) {
                       return dsa_kl_bwd_ex(P(p, 0), P(p, 1), P(p, 2), P(p, 3), P(p, 4), P(p, 5), P(p, 6),
                                            (const int32_t*)P(p, 7), (const float*)P(p, 8), (const float*)P(p, 9),
                                            (const int32_t*)P(p, 10), (const int32_t*)P(p, 11),
                                            (const int32_t*)P(p, 12), (void*)P(p, 13), (void*)P(p, 14),
                                            (void*)P(p, 15), (float*)P(p, 16), v[0], v[1], v[2], v[3], v[4], v[5],
                                            v[6], v[7], v[8], v[9], v[10], v[11], v[12], I32(v, 13), I32(v, 14),
                                            I32(v, 15), I32(v, 16), 0.1f, (void*)0x7f0000, (size_t)v[17], nullptr);
                     }});
  entries.push_back({"dsa_dense_li_softmax_lse",
                     {1, 16, 16, 8, 128, 0, 2},
                     7, {3, 4},
                     [](const Ptrs& p, const Ints& v) {
                       return dsa_dense_li_softmax_lse(P(p, 0), P(p, 1), P(p, 2), (const int32_t*)P(p, 3),
                                                       (const int32_t*)P(p, 4), (float*)P(p, 5), (float*)P(p, 6),
                                                       v[0], v[1], v[2], v[3], v[4], I32(v, 5), I32(v, 6), nullptr);
                     }});
  entries.push_back({"dsa_dense_kl_bwd",
                     {1, 16, 16, 8, 1, 128, 64, 8, 128, 0, 2, 1ll << 30},
                     17, {2, 3, 9, 10, 11, 12},
                     [](const Ptrs& p, const Ints& v) {
                       return dsa_dense_kl_bwd(P(p, 0), P(p, 1), P(p, 2), P(p, 3), P(p, 4), P(p, 5), P(p, 6),
                                               (const float*)P(p, 7), (const float*)P(p, 8), (const float*)P(p, 9),
                                               (const float*)P(p, 10), (const int32_t*)P(p, 11),
                                               (const int32_t*)P(p, 12), (void*)P(p, 13), (void*)P(p, 14),
                                               (void*)P(p, 15), (float*)P(p, 16), v[0], v[1], v[2], v[3], v[4], v[5],
                                               v[6], v[7], v[8], I32(v, 9), I32(v, 10), 0.1f, (void*)0x7f0000,
                                               (size_t)v[11], nullptr);
                     }});
  entries.push_back({"dsa_li_fwd",
                     {1, 4, 256, 8, 1, 128, 64, 4, 256, 3, 0, 0, 0, 2, 1, 1ll << 30},
                     7, {3, 4, 6},
                     [](const Ptrs& p, const Ints& v) {
                       return dsa_li_fwd(P(p, 0), P(p, 1), P(p, 2), (const int32_t*)P(p, 3), (const int32_t*)P(p, 4),
                                         (int32_t*)P(p, 5), (void*)P(p, 6), v[0], v[1], v[2], v[3], v[4], v[5], v[6],
                                         v[7], v[8], I32(v, 9), I32(v, 10), I32(v, 11), I32(v, 12), I32(v, 13),
                                         I32(v, 14), (void*)0x7f0000, (size_t)v[15], nullptr);
                     }});
  entries.push_back({"dsa_li_scores",
                     {1, 4, 256, 8, 1, 128, 4, 256, 3, 0, 0, 0, 2},
                     6, {3, 4},
                     [](const Ptrs& p, const Ints& v) {
                       return dsa_li_scores(P(p, 0), P(p, 1), P(p, 2), (const int32_t*)P(p, 3),
                                            (const int32_t*)P(p, 4), (float*)P(p, 5), v[0], v[1], v[2], v[3], v[4],
                                            v[5], v[6], v[7], I32(v, 8), I32(v, 9), I32(v, 10), I32(v, 11),
                                            I32(v, 12), nullptr);
                     }});
  entries.push_back({"dsa_li_topk_from_scores",
                     {4, 256, 64},
                     3, {2},
                     [](const Ptrs& p, const Ints& v) {
                       return dsa_li_topk_from_scores((const float*)P(p, 0), v[0], v[1], v[2], (int32_t*)P(p, 1),
                                                      (float*)P(p, 2), nullptr);
                     }});
  entries.push_back({"dsa_li_fwd_paged",
                     {1, 4, 8, 1, 128, 64, 4, 4, 64, 4, 3, 0, 0, 2, 1, 1ll << 30},
                     8, {3, 7},
                     [](const Ptrs& p, const Ints& v) {
                       return dsa_li_fwd_paged(P(p, 0), P(p, 1), P(p, 2), (const int32_t*)P(p, 3),
                                               (const int32_t*)P(p, 4), (const int32_t*)P(p, 5), (int32_t*)P(p, 6),
                                               (void*)P(p, 7), v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7], v[8],
                                               v[9], I32(v, 10), I32(v, 11), I32(v, 12), I32(v, 13), I32(v, 14),
                                               (void*)0x7f0000, (size_t)v[15], nullptr);
                     }});
  entries.push_back({"dsa_li_scores_paged",
                     {1, 4, 8, 1, 128, 4, 4, 64, 4, 3, 0, 0, 2},
                     7, {3},
                     [](const Ptrs& p, const Ints& v) {
                       return dsa_li_scores_paged(P(p, 0), P(p, 1), P(p, 2), (const int32_t*)P(p, 3),
                                                  (const int32_t*)P(p, 4), (const int32_t*)P(p, 5), (float*)P(p, 6),
                                                  v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7], v[8], I32(v, 9),
                                                  I32(v, 10), I32(v, 11), I32(v, 12), nullptr);
                     }});
  entries.push_back({"dsa_calib_stream_read",
                     {1 << 20, 0},
                     2, {1},
                     [](const Ptrs& p, const Ints& v) {
                       return dsa_calib_stream_read(P(p, 0), (size_t)v[0], I32(v, 1), (uint32_t*)P(p, 1), nullptr);
                     }});
  for (const Entry& e : entries) sweep(e);

  sweep_size("dsa_sfa_fwd_workspace_size", {32, 128, 512, 2048, 1}, [](const Ints& v) {
    return dsa_sfa_fwd_workspace_size(v[0], v[1], v[2], v[3], (int32_t)v[4]);
  });
  sweep_size("dsa_sfa_bwd_workspace_size", {4096, 4096, 128, 512, 2048, 1, 0}, [](const Ints& v) {
    return dsa_sfa_bwd_workspace_size(v[0], v[1], v[2], v[3], v[4], (int32_t)v[5], (int32_t)v[6]);
  });
  sweep_size("dsa_kl_bwd_workspace_size", {1, 4096, 4096, 2048, 128}, [](const Ints& v) {
    return dsa_kl_bwd_workspace_size(v[0], v[1], v[2], v[3], v[4]);
  });
  sweep_size("dsa_kl_bwd_ex_workspace_size", {4096, 4096, 2048, 128}, [](const Ints& v) {
    return dsa_kl_bwd_ex_workspace_size(v[0], v[1], v[2], v[3]);
  });
  sweep_size("dsa_dense_kl_bwd_workspace_size", {1, 4096, 4096, 128}, [](const Ints& v) {
    return dsa_dense_kl_bwd_workspace_size(v[0], v[1], v[2], v[3]);
  });
  sweep_size("dsa_li_fwd_workspace_size", {32, 1, 32768}, [](const Ints& v) {
    return dsa_li_fwd_workspace_size(v[0], v[1], v[2]);
  });

  // the error message is per thread: a failing call on one thread leaves
  // another thread's message alone
  ++g_cases;
  dsa_sfa_fwd_noalloc(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                      nullptr, 1, 4, 256, 8, 128, 64, 64, 4, 256, 0, 0, 1, 0, kMax, kMax, 0, 0, 0, 0.1f, 0, nullptr);
  const std::string mine = dsa_last_error();
  std::thread([] {
    if (dsa_last_error()[0] != '\0') fail("a new thread starts with a message");
    dsa_li_topk_from_scores(nullptr, 4, 256, 64, nullptr, nullptr, nullptr);
  }).join();
  if (mine != dsa_last_error()) fail("another thread's call changed this thread's message");
  if (mine.empty()) fail("NULL-tensor call left no message");

  printf("%s %d cases, %d failures, abi %d\n", g_fail ? "FAILED" : "OK", g_cases, g_fail, dsa_abi_version());
  return g_fail ? 1 : 0;
}
