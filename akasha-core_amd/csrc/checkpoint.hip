// Reader of akasha-core's V3 checkpoint files (src/nn/checkpoint.rs).
//
// Layout (checkpoint.rs:1-7, 52-96): the 4-byte magic "AKV3", then one
// bincode 1.x V3Body in its little-endian fixint encoding -- fields back to
// back, u32/u64 as 4/8 bytes, Vec<T> as a u64 length then the elements:
//   u32 vocab_size, u32 dim, u32 num_heads, u64 num_layers, u32 seq_len,
//   u32 ffn_hidden, u64 train_step, u32 schedule_step,
//   Vec<Vec<f32>> params    (ModelWeights::params() order),
//   Vec<(Vec<f32>, Vec<f32>)> moments (AdamW (m, v) per param, or empty).
// Host code only: it parses; runtime.hip validates against a model and
// uploads.
#include <stdio.h>
#include <string.h>

#include <string>

#include "akasha_hip.h"
#include "checkpoint.h"

namespace akh {

CkptReader::~CkptReader() {
  if (f_) fclose(f_);
}

bool CkptReader::fail(const std::string& msg) {
  err = msg;
  return false;
}

bool CkptReader::bytes(void* dst, size_t n) {
  if (fread(dst, 1, n, f_) != n) {
    io_error = true;
    return fail(path_ + ": unexpected end of file (truncated checkpoint)");
  }
  return true;
}

bool CkptReader::u32(uint32_t& v) {
  unsigned char b[4];
  if (!bytes(b, 4)) return false;
  v = (uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 | (uint32_t)b[3] << 24;
  return true;
}

bool CkptReader::u64(uint64_t& v) {
  uint32_t lo = 0, hi = 0;
  if (!u32(lo) || !u32(hi)) return false;
  v = (uint64_t)hi << 32 | lo;
  return true;
}

bool CkptReader::open(const char* path) {
  path_ = path ? path : "";
  f_ = path ? fopen(path, "rb") : nullptr;
  if (!f_) {
    io_error = true;
    return fail(path_ + ": cannot open checkpoint");
  }
  if (fseeko(f_, 0, SEEK_END) != 0 || (size_ = ftello(f_)) < 0 || fseeko(f_, 0, SEEK_SET) != 0) {
    io_error = true;
    return fail(path_ + ": cannot read checkpoint");
  }
  char magic[4];
  if (!bytes(magic, 4)) return false;
  if (memcmp(magic, "AKV3", 4) != 0)  // checkpoint.rs:102-109
    return fail(path_ +
                " is not a v3 checkpoint -- migrate it once with: cargo run "
                "--release --bin migrate_checkpoint_v3 -- " + path_);
  return u32(head.vocab_size) && u32(head.dim) && u32(head.num_heads) &&
         u64(head.num_layers) && u32(head.seq_len) && u32(head.ffn_hidden) &&
         u64(head.train_step) && u32(head.schedule_step) && u64(head.num_params);
}

bool CkptReader::tensor_len(uint64_t& n) {
  if (!u64(n)) return false;
  if (n > (uint64_t)1 << 40) return fail(path_ + ": corrupt tensor length");
  return true;
}

bool CkptReader::floats(float* dst, uint64_t n) {
  // The file is little-endian f32 (checkpoint.rs:88-96); so is every host
  // this library is built for.
  return bytes(dst, (size_t)n * sizeof(float));
}

bool CkptReader::skip_floats(uint64_t n) {
  const off_t pos = ftello(f_);
  const off_t end = pos + (off_t)(n * sizeof(float));
  if (pos < 0 || end > size_ || fseeko(f_, end, SEEK_SET) != 0) {
    io_error = true;
    return fail(path_ + ": unexpected end of file (truncated checkpoint)");
  }
  return true;
}

bool CkptReader::at_end() {
  const int c = fgetc(f_);
  if (c == EOF) return true;
  ungetc(c, f_);
  return false;
}

}  // namespace akh
