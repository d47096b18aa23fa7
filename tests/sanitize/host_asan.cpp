// AddressSanitizer + UBSan driver for host-side runtime code: the packers
// and their inverse on ragged shapes with exactly sized buffers, the JSON
// parser on mutated inputs, and the schedule loader on malformed files.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <string>
#include <vector>

#include "runtime/json.h"
#include "runtime/packed_layout.h"
#include "runtime/schedule.h"

int main(int argc, char** argv) {
  // Packers: exact-size allocations so any overrun is reported.
  const int64_t shapes[][3] = {{1, 1, 64}, {64, 128, 64}, {65, 129, 32}, {200, 300, 48},
                               {1000, 17, 64}, {3, 1000, 1}};
  for (auto& sh : shapes) {
    const int64_t K = sh[0], N = sh[1], BK = sh[2];
    std::vector<uint16_t> w(K * N);
    for (size_t i = 0; i < w.size(); ++i) w[i] = (uint16_t)(i * 2654435761u >> 16);
    std::vector<uint16_t> ref((K + BK - 1) / BK * BK * N);
    llk::packReferenceLayout(w.data(), K, N, N, BK, ref.data());
    std::vector<uint8_t> dev(llk::deviceLayoutBytes(K, N));
    llk::packDeviceLayout(w.data(), K, N, N, dev.data());
    std::vector<uint16_t> back(K * N);
    llk::unpackDeviceLayout(dev.data(), K, N, back.data(), N);
    if (back != w) {
      std::printf("unpack(pack(W)) != W for K=%ld N=%ld\n", (long)K, (long)N);
      return 1;
    }
  }
  // JSON parser: the DB file and every single-byte truncation / mutation.
  std::string db;
  if (argc > 1) {
    std::ifstream f(argv[1]);
    db.assign(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
  }
  if (db.empty()) db = "{\"entries\": [{\"operation\": \"fused_swiglu\"}]}";
  llk::json::Value v;
  if (!llk::json::parse(db, &v)) {
    std::printf("DB does not parse\n");
    return 1;
  }
  for (size_t cut = 0; cut < db.size(); cut += 7) (void)llk::json::parse(db.substr(0, cut), &v);
  const char junk[] = "{}[]\",:0-1e+x\\tu";
  for (size_t i = 0; i < db.size(); i += 3) {
    std::string m = db;
    m[i] = junk[i % (sizeof(junk) - 1)];
    (void)llk::json::parse(m, &v);
  }
  // Schedule loader on malformed files.
  const std::string tmp = std::string(std::getenv("TMPDIR") ? std::getenv("TMPDIR") : "/tmp") +
                          "/llk_asan_db.json";
  const char* bad[] = {"", "{", "[]", "{\"entries\": 3}", "{\"entries\": [{}]}",
                       "{\"entries\": [{\"operation\": \"fused_swiglu\", \"shape\": {\"M_bucket\": "
                       "\"x\"}}]}",
                       "{\"entries\": [{\"operation\": \"fused_swiglu\", \"shape\": {\"M_bucket\": "
                       "0, \"N\": 1, \"K\": 1}, \"schedule\": {\"BM\": 1e99}}]}"};
  for (const char* b : bad) {
    std::ofstream(tmp) << b;
    bool ok = true;
    (void)llk::loadScheduleDB(tmp, 0, "fused_swiglu", &ok);
  }
  std::remove(tmp.c_str());
  std::printf("host_asan ok\n");
  return 0;
}
