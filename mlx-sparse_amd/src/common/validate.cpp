// validate.cpp - status-to-exception mapping of the C++ primitive layer.
#include "common/validate.h"

#include <new>

namespace msx {

void throw_status(msx_status st, const char *op) {
  const std::string msg = std::string(msx_last_error());
  const std::string text = msg.empty() ? std::string(op) + " failed." : msg;
  switch (st) {
  case MSX_EINVAL: throw std::invalid_argument(text);
  case MSX_ENOMEM: throw std::bad_alloc();
  case MSX_ETYPE:
  case MSX_EHIP:
  default: throw std::runtime_error(text);
  }
}

}  // namespace msx
