// Internal reader of V3 checkpoint files (src/nn/checkpoint.rs), used by
// akh_checkpoint_info and akh_model_load_checkpoint in runtime.hip.
#pragma once

#include <stdint.h>
#include <stdio.h>
#include <sys/types.h>

#include <string>

namespace akh {

struct CkptHeader {
  uint32_t vocab_size = 0, dim = 0, num_heads = 0;
  uint64_t num_layers = 0;
  uint32_t seq_len = 0, ffn_hidden = 0;
  uint64_t train_step = 0;
  uint32_t schedule_step = 0;
  uint64_t num_params = 0;
};

class CkptReader {
 public:
  ~CkptReader();
  // Opens the file, checks the magic and reads the header up to the
  // parameter count.  On failure `err` says why and `io_error` tells a file
  // that cannot be read from one that is not a V3 checkpoint.
  bool open(const char* path);
  bool tensor_len(uint64_t& n);
  bool floats(float* dst, uint64_t n);
  bool skip_floats(uint64_t n);
  bool u64(uint64_t& v);
  bool at_end();

  CkptHeader head;
  std::string err;
  bool io_error = false;

 private:
  bool fail(const std::string& msg);
  bool bytes(void* dst, size_t n);
  bool u32(uint32_t& v);

  FILE* f_ = nullptr;
  off_t size_ = 0;
  std::string path_;
};

}  // namespace akh
