// Drives sh::plan_eviction (strata-rs_amd/csrc/store.hpp) from text on stdin,
// one case per line:
//   budget incoming call  key:bytes:used:pin  key:bytes:used:pin ...
// and prints, per case, "ok v1 v2 ..." (the victims in eviction order) or
// "oom".
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <sstream>
#include <string>
#include <vector>

#include "../strata-rs_amd/csrc/store.hpp"

int main() {
  std::string line;
  char buf[4096];
  while (fgets(buf, sizeof buf, stdin)) {
    std::istringstream in(buf);
    unsigned long long budget = 0, incoming = 0, call = 0;
    if (!(in >> budget >> incoming >> call)) continue;
    std::vector<sh::StoreEntry> entries;
    unsigned long long total = 0;
    std::string tok;
    while (in >> tok) {
      unsigned long long k, b, u, p;
      if (sscanf(tok.c_str(), "%llu:%llu:%llu:%llu", &k, &b, &u, &p) != 4) return 2;
      entries.push_back({k, b, u, p});
      total += b;
    }
    std::vector<uint64_t> victims;
    if (sh::plan_eviction(entries, total, budget, incoming, call, &victims)) {
      printf("ok");
      for (uint64_t v : victims) printf(" %llu", (unsigned long long)v);
      printf("\n");
    } else {
      printf("oom\n");
    }
  }
  return 0;
}
