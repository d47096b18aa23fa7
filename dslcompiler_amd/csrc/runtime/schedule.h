// schedule.h -- M-bucket classification and schedule-database lookup.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace llk {

// ScheduleEntry (ScheduleLoader.h:23-31).
struct ScheduleEntry {
  int64_t BM{0}, BN{0}, BK{0};
  int64_t VM{0}, VN{0};
  int64_t vector_width{0};
  int64_t num_threads{1};
  int64_t grain_size{1};
  std::string parallel_axis;
};

// classifyM (ScheduleLoader.cpp:19-29): {1}->0, [2,4]->1, [5,16]->2,
// [17,64]->3, >=65->4; M <= 0 lands in bucket 1 like the reference.
int classifyM(int64_t M);

// loadScheduleDB (ScheduleLoader.cpp:31-98): every entry whose "operation"
// equals opName and whose shape.M_bucket equals M_bucket, in file order.
// shape.N and shape.K must be present integers but are NOT compared (the
// reference ignores its N/K arguments); "target" is ignored too.  Missing
// schedule integers default to 0 (BM..vector_width) or 1 (num_threads,
// grain_size).  *ok is false when the file cannot be read or parsed.
std::vector<ScheduleEntry> loadScheduleDB(const std::string& path, int M_bucket,
                                          const std::string& opName, bool* ok);

// selectBest (ScheduleSelection.cpp:46-67): first match, else the built-in
// default {BM 8, BN 32, BK 32, VM 1, VN 4, vector_width 8, threads 4,
// grain 1, axis "n"}.
ScheduleEntry selectBest(const std::vector<ScheduleEntry>& matches);

}  // namespace llk
