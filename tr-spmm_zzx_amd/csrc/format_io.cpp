// Format cache files (trs_format_write / trs_format_read in include/trspmm.h).
//
// Layout, little-endian:
//   Header  magic "TRSFMT01", version, slot count (32), rows, window, canonical flag, reserved,
//           build time (double), numel of each of the 32 slots (int64)
//   Data    each slot's elements in slot order, every slot padded to a multiple of 8 bytes
//   Trailer 64-bit FNV-1a over the 8-byte words of header + data
// The reader checks magic, version, slot count, that the sizes account for the file exactly and
// the checksum, and only then fills a trs_format.  Indices are not validated here: plan creation
// validates every index it lowers, as it does for freshly built formats.
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "format.hpp"

namespace {

constexpr char kMagic[8] = {'T', 'R', 'S', 'F', 'M', 'T', '0', '1'};
constexpr uint32_t kVersion = 1;
constexpr int kSlots = 32;

struct Header {
  char magic[8];
  uint32_t version;
  uint32_t slots;
  int32_t rows;
  int32_t window;
  int32_t canonical;
  int32_t reserved;
  double elapsed;
  int64_t numel[kSlots];
};
static_assert(sizeof(Header) == 40 + 8 * kSlots, "packed header");

// Calls fn(vector&) for the slot's storage (same numbering as trs_format_slot).
template <class Fn>
void with_slot(trs_format& F, int slot, Fn&& fn) {
  switch (slot) {
    case 0: fn(F.t_rowoff); break;     case 1: fn(F.t_blockoff); break;  case 2: fn(F.t_col); break;
    case 3: fn(F.t_val); break;        case 4: fn(F.t_winrow); break;    case 5: fn(F.t_atomic); break;
    case 6: fn(F.t_bin); break;        case 7: fn(F.c_off); break;       case 8: fn(F.c_row); break;
    case 9: fn(F.c_atomic); break;     case 10: fn(F.c_col); break;      case 11: fn(F.c_val); break;
    case 12: fn(F.cs_off); break;      case 13: fn(F.cs_row); break;     case 14: fn(F.cs_atomic); break;
    case 15: fn(F.cs_col); break;      case 16: fn(F.cs_val); break;     case 17: fn(F.s_col); break;
    case 18: fn(F.s_mask); break;      case 19: fn(F.s_val); break;      case 20: fn(F.s_pos); break;
    case 21: fn(F.s_win); break;       case 22: fn(F.s_offsets); break;  case 23: fn(F.tile_win); break;
    case 24: fn(F.tile_group); break;  case 25: fn(F.tile_cols); break;  case 26: fn(F.packed_a); break;
    case 27: fn(F.packed_meta); break; case 28: fn(F.win_tile_off); break;
    case 29: fn(F.spill_row); break;   case 30: fn(F.spill_col); break;  default: fn(F.spill_val); break;
  }
}

size_t pad8(size_t b) { return (b + 7) & ~size_t(7); }
constexpr unsigned char kZeros[8] = {0, 0, 0, 0, 0, 0, 0, 0};

// FNV-1a with 8-byte words as its symbols; every block it sees is a multiple of 8 bytes (slots
// are checksummed together with their padding).
struct Fnv {
  uint64_t h = 1469598103934665603ull;
  void add(const void* p, size_t n) {
    const unsigned char* b = static_cast<const unsigned char*>(p);
    for (size_t i = 0; i + 8 <= n; i += 8) {
      uint64_t w;
      std::memcpy(&w, b + i, 8);
      h = (h ^ w) * 1099511628211ull;
    }
  }
};

int io_error(const std::string& msg) {
  trs::set_error(msg);
  return TRS_EIO;
}

}  // namespace

extern "C" {

int trs_format_write(const trs_format* F, const char* path) {
  if (!F || !path) {
    trs::set_error("trs_format_write: NULL argument");
    return TRS_EINVAL;
  }
  trs_format& M = const_cast<trs_format&>(*F);   // with_slot only reads here
  Header h;
  std::memset(&h, 0, sizeof h);
  std::memcpy(h.magic, kMagic, 8);
  h.version = kVersion;
  h.slots = kSlots;
  h.rows = F->rows;
  h.window = F->window;
  h.canonical = F->canonical ? 1 : 0;
  h.elapsed = F->elapsed;
  for (int s = 0; s < kSlots; ++s) with_slot(M, s, [&](auto& v) { h.numel[s] = (int64_t)v.size(); });

  // write to a temporary name, then rename: a reader never sees a partial file
  const std::string tmp = std::string(path) + ".tmp";
  std::FILE* fp = std::fopen(tmp.c_str(), "wb");
  if (!fp) return io_error(std::string("trs_format_write: cannot open ") + tmp);
  Fnv sum;
  bool ok = std::fwrite(&h, sizeof h, 1, fp) == 1;
  sum.add(&h, sizeof h);
  for (int s = 0; s < kSlots && ok; ++s) {
    with_slot(M, s, [&](auto& v) {
      const size_t bytes = v.size() * sizeof(v[0]);
      const size_t body = bytes & ~size_t(7), pad = pad8(bytes) - bytes;
      if (bytes && std::fwrite(v.data(), 1, bytes, fp) != bytes) ok = false;
      if (pad && std::fwrite(kZeros, 1, pad, fp) != pad) ok = false;
      sum.add(v.data(), body);
      if (pad) {   // last partial word, zero-padded as written
        unsigned char tail[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        std::memcpy(tail, reinterpret_cast<const unsigned char*>(v.data()) + body, bytes - body);
        sum.add(tail, 8);
      }
    });
  }
  ok = ok && std::fwrite(&sum.h, sizeof sum.h, 1, fp) == 1;
  ok = (std::fclose(fp) == 0) && ok;
  if (!ok || std::rename(tmp.c_str(), path) != 0) {
    std::remove(tmp.c_str());
    return io_error(std::string("trs_format_write: write failed for ") + path);
  }
  return TRS_OK;
}

int trs_format_read(const char* path, trs_format** out) {
  if (!path || !out) {
    trs::set_error("trs_format_read: NULL argument");
    return TRS_EINVAL;
  }
  *out = nullptr;
  std::FILE* fp = std::fopen(path, "rb");
  if (!fp) return io_error(std::string("trs_format_read: cannot open ") + path);
  struct Closer { std::FILE* f; ~Closer() { std::fclose(f); } } closer{fp};
  if (std::fseek(fp, 0, SEEK_END) != 0) return io_error("trs_format_read: cannot seek");
  const long long file_size = std::ftell(fp);
  std::rewind(fp);
  Header h;
  if (file_size < (long long)(sizeof h + 8) || std::fread(&h, sizeof h, 1, fp) != 1)
    return io_error("trs_format_read: file too short for a format");
  if (std::memcmp(h.magic, kMagic, 8) != 0) return io_error("trs_format_read: not a format cache file");
  if (h.version != kVersion || h.slots != (uint32_t)kSlots)
    return io_error("trs_format_read: unsupported format file version");
  if (h.window < 1 || h.window > 32 || h.rows < 0) return io_error("trs_format_read: bad header fields");

  trs_format probe;
  size_t need = sizeof h;
  for (int s = 0; s < kSlots; ++s) {
    if (h.numel[s] < 0 || h.numel[s] > ((int64_t)1 << 40)) return io_error("trs_format_read: bad slot size");
    with_slot(probe, s, [&](auto& v) { need += pad8((size_t)h.numel[s] * sizeof(v[0])); });
  }
  if ((long long)need + 8 != file_size) return io_error("trs_format_read: file size does not match its header");

  trs_format* F = new (std::nothrow) trs_format();
  if (!F) {
    trs::set_error("trs_format_read: out of memory");
    return TRS_ENOMEM;
  }
  F->rows = h.rows;
  F->window = h.window;
  F->canonical = h.canonical != 0;
  F->elapsed = h.elapsed;
  Fnv sum;
  sum.add(&h, sizeof h);
  bool ok = true;
  try {
    for (int s = 0; s < kSlots && ok; ++s) {
      with_slot(*F, s, [&](auto& v) {
        const size_t bytes = (size_t)h.numel[s] * sizeof(v[0]);
        const size_t body = bytes & ~size_t(7), pad = pad8(bytes) - bytes;
        v.resize((size_t)h.numel[s]);
        if (bytes && std::fread(v.data(), 1, bytes, fp) != bytes) ok = false;
        unsigned char tail[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (pad && std::fread(tail + (bytes - body), 1, pad, fp) != pad) ok = false;
        sum.add(v.data(), body);
        if (pad) {
          std::memcpy(tail, reinterpret_cast<const unsigned char*>(v.data()) + body, bytes - body);
          sum.add(tail, 8);
        }
      });
    }
  } catch (const std::bad_alloc&) {
    delete F;
    trs::set_error("trs_format_read: out of memory");
    return TRS_ENOMEM;
  }
  uint64_t stored = 0;
  if (!ok || std::fread(&stored, 8, 1, fp) != 1) {
    delete F;
    return io_error("trs_format_read: short read");
  }
  if (stored != sum.h) {
    delete F;
    return io_error("trs_format_read: checksum mismatch (corrupted file)");
  }
  *out = F;
  return TRS_OK;
}

}  // extern "C"
