// schedule.cpp -- restatement of the reference's schedule lookup
// (ScheduleLoader.cpp:19-98, ScheduleSelection.cpp:46-67) over json.h.
#include "schedule.h"

#include <fstream>
#include <sstream>

#include "json.h"

namespace llk {

int classifyM(int64_t M) {
  if (M == 1) return 0;
  if (M <= 4) return 1;
  if (M <= 16) return 2;
  if (M <= 64) return 3;
  return 4;
}

std::vector<ScheduleEntry> loadScheduleDB(const std::string& path, int M_bucket,
                                          const std::string& opName, bool* ok) {
  std::vector<ScheduleEntry> matches;
  if (ok) *ok = false;
  std::ifstream f(path, std::ios::binary);
  if (!f) return matches;
  std::stringstream ss;
  ss << f.rdbuf();
  json::Value root;
  if (!json::parse(ss.str(), &root)) return matches;
  if (ok) *ok = true;
  if (root.kind != json::Value::Object) return matches;
  const json::Value* entries = root.getArray("entries");
  if (!entries) return matches;
  for (const json::Value& e : entries->arr) {
    if (e.kind != json::Value::Object) continue;
    const std::string* op = e.getString("operation");
    if (!op || *op != opName) continue;
    const json::Value* shape = e.getObject("shape");
    if (!shape) continue;
    int64_t bucket, n, k;
    if (!shape->getInteger("M_bucket", &bucket) || bucket != M_bucket) continue;
    if (!shape->getInteger("N", &n) || !shape->getInteger("K", &k)) continue;
    const json::Value* s = e.getObject("schedule");
    if (!s) continue;
    ScheduleEntry se;
    auto geti = [&](const char* key, int64_t dflt) {
      int64_t v;
      return s->getInteger(key, &v) ? v : dflt;
    };
    se.BM = geti("BM", 0);
    se.BN = geti("BN", 0);
    se.BK = geti("BK", 0);
    se.VM = geti("VM", 0);
    se.VN = geti("VN", 0);
    se.vector_width = geti("vector_width", 0);
    se.num_threads = geti("num_threads", 1);
    se.grain_size = geti("grain_size", 1);
    if (const std::string* ax = s->getString("parallel_axis")) se.parallel_axis = *ax;
    matches.push_back(se);
  }
  return matches;
}

ScheduleEntry selectBest(const std::vector<ScheduleEntry>& matches) {
  if (matches.empty()) {
    ScheduleEntry d;
    d.BM = 8;
    d.BN = 32;
    d.BK = 32;
    d.VM = 1;
    d.VN = 4;
    d.vector_width = 8;
    d.num_threads = 4;
    d.grain_size = 1;
    d.parallel_axis = "n";
    return d;
  }
  return matches.front();
}

}  // namespace llk
