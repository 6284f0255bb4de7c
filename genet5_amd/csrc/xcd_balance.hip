// Per-XCD tile shares of the persistent grouped GEMM launches.
//
// New stage (no reference counterpart).  A persistent launch of 8 x 32
// workgroups cuts its tile list into 8 contiguous ranges, one per XCD (workgroup
// b runs on XCD b % 8).  The XCDs do not run at the same speed: at config 2 the
// gate|up launch's XCDs finish up to 35 us apart, in the same order call after
// call (per-XCD lateness correlates 0.99 between consecutive calls), so equal
// ranges leave the fast XCDs idle at the end.  Here each XCD's share follows its
// measured rate:
//
//   * every workgroup of a balanced launch writes one 64-bit record, (launch tag
//     << 32) | its busy time in 100 MHz ticks, into a small host-mapped buffer
//     of its launch site (one per device, GEMM mode, tile shape and K x Nout);
//   * before the next launch of the site the host reads that buffer; when every
//     record carries one tag of a recent launch, XCD x's rate is its share under
//     that launch's weights over its slowest workgroup's busy time, and the new
//     weights move halfway to shares proportional to those rates;
//   * the weights travel in the kernel arguments (cumulative, summing to
//     kWeightSum), so every workgroup of a launch cuts the same ranges.
//
// Nothing waits: the host uses whatever completed record it finds (usually one
// from a few launches back) and otherwise keeps its weights.  The tile
// partition is valid for any weights and every tile's arithmetic is the same
// whichever workgroup runs it, so outputs do not depend on the split.  Under
// HIP graph capture no buffer is allocated (a site first seen there runs the
// equal split without records), and a captured launch keeps the weights of its
// capture.
#include <algorithm>
#include <mutex>

#include "g5moe_internal.h"

namespace g5moe {

namespace {

constexpr int kSlotsPerXcd = 32;
constexpr int kWorkgroups = 8 * kSlotsPerXcd;
constexpr int kWeightSum = 8192;
constexpr int kMinWeight = kWeightSum / 64;  // no XCD drops below 1/8 of an equal share
constexpr int kHistory = 16;                 // launches whose weights are remembered
constexpr int kMaxSites = 64;

struct Site {
  int dev, site, K, nout;
  bool disabled;
  unsigned long long* host;  // kWorkgroups records (host view)
  unsigned long long* devp;  // the same memory as the kernels address it
  uint32_t seq;              // tag of the last launch
  int w[8];                  // current weights
  int hist[kHistory][8];     // weights of launch tag t at t % kHistory
};

std::mutex g_mu;
Site g_sites[kMaxSites];
int g_nsites = 0;

void cumulative(const int (&w)[8], XcdSplit& xs) {
  xs.w[0] = 0;
  for (int x = 0; x < 8; ++x) xs.w[x + 1] = xs.w[x] + w[x];
}

// New weights from the records of a completed launch, if the buffer holds one.
void update(Site& s) {
  const uint32_t tag = uint32_t(__atomic_load_n(&s.host[0], __ATOMIC_RELAXED) >> 32);
  if (tag == 0 || s.seq - tag >= uint32_t(kHistory)) return;  // none, or too old
  double busy[8] = {};
  for (int b = 0; b < kWorkgroups; ++b) {
    const unsigned long long r = __atomic_load_n(&s.host[b], __ATOMIC_RELAXED);
    if (uint32_t(r >> 32) != tag) return;  // a launch still writing, or several mixed
    const double t = double(uint32_t(r));
    if (t > busy[b & 7]) busy[b & 7] = t;
  }
  const int* used = s.hist[tag % kHistory];
  double rate[8], rsum = 0.0;
  for (int x = 0; x < 8; ++x) {
    if (!(busy[x] > 0.0)) return;
    rate[x] = double(used[x]) / busy[x];
    rsum += rate[x];
  }
  int w[8], sum = 0;
  for (int x = 0; x < 8; ++x) {
    const double target = kWeightSum * rate[x] / rsum;
    w[x] = std::max(kMinWeight, int(0.5 * (s.w[x] + target) + 0.5));
    sum += w[x];
  }
  // exact sum: the remainder goes to the largest weight
  int big = 0;
  for (int x = 1; x < 8; ++x) big = w[x] > w[big] ? x : big;
  w[big] += kWeightSum - sum;
  if (w[big] < kMinWeight) return;
  for (int x = 0; x < 8; ++x) s.w[x] = w[x];
  // this record has been used: later calls wait for a newer one
  __atomic_store_n(&s.host[0], 0ull, __ATOMIC_RELAXED);
}

}  // namespace

XcdSplit xcd_split(int site, unsigned grid, int K, int nout, hipStream_t st) {
  XcdSplit xs{};  // w[8] == 0: the equal split, no records
  if (grid != unsigned(kWorkgroups)) return xs;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return xs;
  std::lock_guard<std::mutex> lock(g_mu);
  Site* s = nullptr;
  for (int i = 0; i < g_nsites; ++i)
    if (g_sites[i].dev == dev && g_sites[i].site == site && g_sites[i].K == K &&
        g_sites[i].nout == nout)
      s = &g_sites[i];
  if (s == nullptr) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (g_nsites == kMaxSites || hipStreamIsCapturing(st, &cap) != hipSuccess ||
        cap != hipStreamCaptureStatusNone)
      return xs;
    s = &g_sites[g_nsites++];
    *s = Site{};
    s->dev = dev;
    s->site = site;
    s->K = K;
    s->nout = nout;
    for (int x = 0; x < 8; ++x) s->w[x] = kWeightSum / 8;
    int can_map = 0;
    void* h = nullptr;
    if (hipDeviceGetAttribute(&can_map, hipDeviceAttributeCanMapHostMemory, dev) != hipSuccess ||
        can_map == 0) {
      (void)hipGetLastError();
      s->disabled = true;  // the kernels could not address a host buffer: equal split
    } else if (hipHostMalloc(&h, kWorkgroups * sizeof(unsigned long long),
                             hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess) {
      (void)hipGetLastError();
      s->disabled = true;
    } else {
      s->host = static_cast<unsigned long long*>(h);
      for (int b = 0; b < kWorkgroups; ++b) s->host[b] = 0;
      void* d = nullptr;
      if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess) {
        (void)hipGetLastError();
        s->disabled = true;
      } else {
        s->devp = static_cast<unsigned long long*>(d);
      }
    }
  }
  if (s->disabled) return xs;
  update(*s);
  s->seq = s->seq + 1 == 0 ? 1 : s->seq + 1;  // tag 0 marks an empty buffer
  for (int x = 0; x < 8; ++x) s->hist[s->seq % kHistory][x] = s->w[x];
  cumulative(s->w, xs);
  xs.probe = s->devp;
  xs.seq = s->seq;
  return xs;
}

}  // namespace g5moe
