// A process-local mapping of the shared command queue segment.  The
// ext_ipc_queue side and the aggregator each hold their own mapping, as the
// reference's two extension modules do.
#pragma once

#include <string>

#include "ipc_layout.h"

namespace swl {

struct QueueMap {
  void* base = nullptr;
  size_t bytes = 0;
  std::string name;
  bool owner = false;
  Control* ctrl = nullptr;
  Command* ring = nullptr;
  int capacity = 0;

  int create(int capacity, int max_tickets);
  int open(const char* shm_name, int capacity);
  void close_map();
};

extern QueueMap g_queue;

}  // namespace swl
