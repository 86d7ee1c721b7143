// marisa/base.h -- basic types, error codes and build flags of the drop-in
// C++ surface.  Values match the reference's include/marisa/base.h so code
// written against it compiles and means the same thing (error codes
// :52-90, config flags :100-156, Label/UInt32 :186-191).
#ifndef MARISA_BASE_H_
#define MARISA_BASE_H_

#include <stdint.h>

#include <cstddef>
#include <exception>
#include <string>
#include <utility>

typedef enum marisa_error_code_ {
  MARISA_OK = 0,
  MARISA_STATE_ERROR = 1,
  MARISA_NULL_ERROR = 2,
  MARISA_BOUND_ERROR = 3,
  MARISA_RANGE_ERROR = 4,
  MARISA_CODE_ERROR = 5,
  MARISA_RESET_ERROR = 6,
  MARISA_SIZE_ERROR = 7,
  MARISA_MEMORY_ERROR = 8,
  MARISA_IO_ERROR = 9,
  MARISA_FORMAT_ERROR = 10,
} marisa_error_code;

typedef enum marisa_num_tries_ {
  MARISA_MIN_NUM_TRIES = 0x00001,
  MARISA_MAX_NUM_TRIES = 0x0007F,
  MARISA_DEFAULT_NUM_TRIES = 0x00003,
} marisa_num_tries;

typedef enum marisa_cache_level_ {
  MARISA_HUGE_CACHE = 0x00080,
  MARISA_LARGE_CACHE = 0x00100,
  MARISA_NORMAL_CACHE = 0x00200,
  MARISA_SMALL_CACHE = 0x00400,
  MARISA_TINY_CACHE = 0x00800,
  MARISA_DEFAULT_CACHE = MARISA_NORMAL_CACHE
} marisa_cache_level;

typedef enum marisa_tail_mode_ {
  MARISA_TEXT_TAIL = 0x01000,
  MARISA_BINARY_TAIL = 0x02000,
  MARISA_DEFAULT_TAIL = MARISA_TEXT_TAIL,
} marisa_tail_mode;

typedef enum marisa_node_order_ {
  MARISA_LABEL_ORDER = 0x10000,
  MARISA_WEIGHT_ORDER = 0x20000,
  MARISA_DEFAULT_ORDER = MARISA_WEIGHT_ORDER,
} marisa_node_order;

typedef enum marisa_config_mask_ {
  MARISA_NUM_TRIES_MASK = 0x0007F,
  MARISA_CACHE_LEVEL_MASK = 0x00F80,
  MARISA_TAIL_MODE_MASK = 0x0F000,
  MARISA_NODE_ORDER_MASK = 0xF0000,
  MARISA_CONFIG_MASK = 0xFFFFF
} marisa_config_mask;

namespace marisa {

typedef uint8_t UInt8;
typedef uint16_t UInt16;
typedef uint32_t UInt32;
typedef uint64_t UInt64;
typedef ::marisa_error_code ErrorCode;
typedef ::marisa_tail_mode TailMode;
typedef ::marisa_node_order NodeOrder;
typedef UInt32 Label;

// Thrown on every host-side error (the reference's marisa::Exception,
// include/marisa/exception.h:12-55); what() carries the message.
class Exception : public std::exception {
 public:
  Exception(ErrorCode code, std::string message)
      : code_(code), message_(std::move(message)) {}
  ErrorCode error_code() const { return code_; }
  const char* error_message() const { return message_.c_str(); }
  const char* what() const noexcept override { return message_.c_str(); }

 private:
  ErrorCode code_;
  std::string message_;
};

}  // namespace marisa

#endif  // MARISA_BASE_H_
