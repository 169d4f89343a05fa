// Host-side helpers shared by the drivers (conv_lab, vendor_lab): the
// workload table of the reference's workloads.csv:1 schema, read at run
// time (the reference compiled one case per binary: gen_case.py:15-36 +
// Makefile:41-47), fatal errors, and the executable's directory.
#pragma once

#include <stdlib.h>
#include <unistd.h>

#include <fstream>
#include <iostream>
#include <map>
#include <string>
#include <vector>

#include "i8conv.h"

namespace i8conv_host {

[[noreturn]] inline void fail(const std::string &what) {
  std::cerr << what << '\n';
  std::exit(EXIT_FAILURE);
}

// ---- workload table (schema of the reference's workloads.csv:1) ----------

inline const char *const kFields[] = {"n", "h", "w", "c", "k", "r", "s",
                                     "pad_h", "pad_w", "stride_h", "stride_w",
                                     "dilation_h", "dilation_w"};

inline std::vector<std::string> split_csv_line(const std::string &line) {
  std::vector<std::string> out;
  std::string cur;
  for (char ch : line) {
    if (ch == ',') {
      out.push_back(cur);
      cur.clear();
    } else if (ch != '\r' && ch != '\n') {
      cur.push_back(ch);
    }
  }
  out.push_back(cur);
  return out;
}

// Looks a case up by name (gen_case.py:20-27): unknown case and missing
// columns are fatal, with the same messages.
inline i8conv_shape load_case(const std::string &path, const std::string &name) {
  std::ifstream in(path);
  if (!in) fail("cannot open workload table " + path);
  std::string line;
  if (!std::getline(in, line)) fail(path + " is empty");
  const std::vector<std::string> header = split_csv_line(line);
  std::map<std::string, size_t> col;
  for (size_t i = 0; i < header.size(); ++i) col[header[i]] = i;
  if (!col.count("name")) fail(path + " is missing columns: name");
  while (std::getline(in, line)) {
    if (line.empty()) continue;
    const std::vector<std::string> row = split_csv_line(line);
    if (col["name"] >= row.size() || row[col["name"]] != name) continue;
    std::vector<std::string> missing;
    for (const char *f : kFields)
      if (!col.count(f)) missing.push_back(f);
    if (!missing.empty()) {
      std::string m;
      for (size_t i = 0; i < missing.size(); ++i) m += (i ? ", " : "") + missing[i];
      fail(path + " is missing columns: " + m);
    }
    int v[13];
    for (int i = 0; i < 13; ++i) {
      const size_t c = col[kFields[i]];
      if (c >= row.size()) fail("short row for case '" + name + "' in " + path);
      char *end = nullptr;
      const long x = strtol(row[c].c_str(), &end, 10);
      if (end == row[c].c_str() || *end != '\0')
        fail("bad value '" + row[c] + "' for " + kFields[i] + " in case '" + name + "'");
      v[i] = int(x);
    }
    return i8conv_shape{v[0], v[1], v[2], v[3], v[4], v[5], v[6],
                        v[7], v[8], v[9], v[10], v[11], v[12]};
  }
  fail("unknown case '" + name + "' in " + path);
}

inline std::string exe_dir() {
  char buf[4096];
  const ssize_t n = readlink("/proc/self/exe", buf, sizeof(buf) - 1);
  if (n <= 0) return ".";
  buf[n] = '\0';
  std::string p(buf);
  const size_t slash = p.rfind('/');
  return slash == std::string::npos ? "." : p.substr(0, slash);
}

}  // namespace i8conv_host
