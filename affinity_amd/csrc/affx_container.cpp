// The .aff container, read on the host: one read-only mapping of the file, the header and
// section checks, the layer table, O(1) expert addressing and the __codebook tensor, then the
// upload of a layer's experts into the device layout.
//
// The on-disk structures are the reference's format (src/format/aff_format.h:138-226: header 192
// bytes, matrix descriptor 72, layer descriptor 240, tensor entry 208, all little-endian), written
// out here field by field so the bytes of a container the reference's aff-quantize wrote are read
// as they are. Checks: the reader's own (src/format/aff_reader.cpp:56-118: magic, version, file
// size, every section inside the file, every layer's experts inside the pool) and the load-time
// ones of the expert tier (src/gpu/static_placement.hip:918-951, src/engine/model.cpp:335-357):
// the quad format in every matrix, the plane geometry of compute_expert_layout, a 2048-dword
// codebook whose every byte has stored exponent 1..7.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <new>

#include "affx_common.h"

namespace {

constexpr char kAffMagic[8] = {'A', 'F', 'F', 'I', 'N', 'I', 'T', 'Y'};
constexpr uint32_t kAffVersion = 1;
constexpr uint32_t kAffQuad = 33;  // AFF_Q2P875_Q4
constexpr uint32_t kAffF32 = 0;
constexpr int kTensorName = 128;

struct DiskMatrix {
  uint64_t rows, cols;
  uint32_t quant, pad;
  uint64_t data_off, data_size, scale_off, scale_size, rscale_off, rscale_size;
};
struct DiskLayer {
  uint32_t layer, n_experts;
  uint64_t base_off, stride;
  DiskMatrix gate, up, down;
};
struct DiskTensor {
  char name[kTensorName];
  DiskMatrix desc;
  uint64_t blob_off;
};
struct DiskHeader {
  char magic[8];
  uint32_t version, flags;
  uint64_t meta_off, meta_size;
  uint64_t tensor_dir_off, tensor_count, tensor_data_off, tensor_data_size;
  uint64_t layer_dir_off, layer_count;
  uint64_t expert_pool_off, expert_pool_size;
  uint64_t profile_off, profile_size;
  uint64_t file_size;
  uint8_t reserved[72];
};
static_assert(sizeof(DiskMatrix) == 72, "matrix descriptor is 72 bytes on disk");
static_assert(sizeof(DiskLayer) == 240, "layer descriptor is 240 bytes on disk");
static_assert(sizeof(DiskTensor) == 208, "tensor entry is 208 bytes on disk");
static_assert(sizeof(DiskHeader) == 192, "header is 192 bytes on disk");

}  // namespace

struct affx_container {
  int fd = -1;
  const uint8_t* map = nullptr;
  uint64_t size = 0;
  const DiskHeader* hdr = nullptr;
  const DiskLayer* layers = nullptr;
  const uint8_t* pool = nullptr;
  uint32_t codebook[2048];
};

using namespace affx;

namespace {

void close_container(affx_container* c) {
  if (!c) return;
  if (c->map) munmap(const_cast<uint8_t*>(c->map), c->size);
  if (c->fd >= 0) ::close(c->fd);
  delete c;
}

bool in_file(const affx_container* c, uint64_t off, uint64_t n) { return off <= c->size && n <= c->size - off; }

// The reference's three quad-format matrices at (hidden, inter): shapes and plane geometry.
bool layer_matches(const DiskLayer& L, uint64_t* hidden, uint64_t* inter) {
  const uint64_t I = L.gate.rows, H = L.gate.cols;
  if (L.up.rows != I || L.up.cols != H || L.down.rows != H || L.down.cols != I) return false;
  uint64_t off[9], size[9];
  const uint64_t stride = affx_expert_layout(H, I, off, size);
  const DiskMatrix* m[3] = {&L.gate, &L.up, &L.down};
  for (int i = 0; i < 3; ++i) {
    if (m[i]->quant != kAffQuad) return false;
    if (m[i]->data_off != off[3 * i] || m[i]->data_size != size[3 * i] || m[i]->scale_off != off[3 * i + 1] ||
        m[i]->scale_size != size[3 * i + 1] || m[i]->rscale_off != off[3 * i + 2] ||
        m[i]->rscale_size != size[3 * i + 2])
      return false;
  }
  if (L.stride < stride) return false;
  *hidden = H;
  *inter = I;
  return true;
}

}  // namespace

extern "C" {

int affx_container_open(const char* path, affx_container** out) {
  if (!path || !out) return set_error(AFFX_ERR_ARG, "container_open: null argument");
  *out = nullptr;
  affx_container* c = new (std::nothrow) affx_container();
  if (!c) return set_error(AFFX_ERR_ARG, "container_open: out of memory");
  auto fail = [&](const char* fmt, auto... a) {
    close_container(c);
    return set_error(AFFX_ERR_ARG, fmt, a...);
  };
  c->fd = ::open(path, O_RDONLY);
  if (c->fd < 0) return fail("container_open: %s: %s", path, std::strerror(errno));
  struct stat st {};
  if (fstat(c->fd, &st) != 0) return fail("container_open: fstat: %s", std::strerror(errno));
  c->size = (uint64_t)st.st_size;
  if (c->size < sizeof(DiskHeader)) return fail("container_open: file too small to hold a header");
  void* m = mmap(nullptr, c->size, PROT_READ, MAP_SHARED, c->fd, 0);
  if (m == MAP_FAILED) return fail("container_open: mmap: %s", std::strerror(errno));
  c->map = (const uint8_t*)m;
  c->hdr = (const DiskHeader*)c->map;
  const DiskHeader& h = *c->hdr;
  if (std::memcmp(h.magic, kAffMagic, 8) != 0) return fail("container_open: bad magic, not a .aff file");
  if (h.version != kAffVersion) return fail("container_open: version %u, expected %u", h.version, kAffVersion);
  if (h.file_size != c->size)
    return fail("container_open: truncated: the header says %llu bytes, the file has %llu",
                (unsigned long long)h.file_size, (unsigned long long)c->size);
  if (h.layer_count > (1u << 20) || h.tensor_count > (1u << 24) ||
      !in_file(c, h.meta_off, h.meta_size) || !in_file(c, h.layer_dir_off, h.layer_count * sizeof(DiskLayer)) ||
      !in_file(c, h.tensor_dir_off, h.tensor_count * sizeof(DiskTensor)) ||
      !in_file(c, h.tensor_data_off, h.tensor_data_size) || !in_file(c, h.expert_pool_off, h.expert_pool_size) ||
      !in_file(c, h.profile_off, h.profile_size))
    return fail("container_open: corrupt header: a section lies outside the file");
  c->layers = (const DiskLayer*)(c->map + h.layer_dir_off);
  c->pool = c->map + h.expert_pool_off;
  for (uint64_t i = 0; i < h.layer_count; ++i) {
    const DiskLayer& L = c->layers[i];
    // (the experts' extent by division: n_experts * stride can wrap for a corrupt stride)
    if (L.stride == 0 || L.n_experts > AFFX_MAX_EXPERTS || L.base_off > h.expert_pool_size ||
        (L.n_experts > 0 && L.stride > (h.expert_pool_size - L.base_off) / L.n_experts))
      return fail("container_open: corrupt layer descriptor %llu", (unsigned long long)i);
    uint64_t H = 0, I = 0;
    if (!layer_matches(L, &H, &I))
      return fail("container_open: layer %llu is not %s quad-format experts with the plane geometry of its "
                  "shape (quant ids %u %u %u)", (unsigned long long)i, "2.875-bpw", L.gate.quant, L.up.quant,
                  L.down.quant);
  }
  // the codebook: one f32-declared tensor of 2048 entries holding the packed dwords
  const DiskTensor* t = (const DiskTensor*)(c->map + h.tensor_dir_off);
  const DiskTensor* cb = nullptr;
  for (uint64_t i = 0; i < h.tensor_count && !cb; ++i)
    if (strnlen(t[i].name, kTensorName) == 10 && std::memcmp(t[i].name, "__codebook", 10) == 0) cb = &t[i];
  if (!cb) return fail("container_open: no __codebook tensor");
  if (cb->desc.rows * cb->desc.cols != 2048 || cb->desc.quant != kAffF32 || cb->desc.data_size < 2048 * 4 ||
      cb->blob_off > h.tensor_data_size || cb->desc.data_off > h.tensor_data_size - cb->blob_off ||
      2048 * 4 > h.tensor_data_size - cb->blob_off - cb->desc.data_off)
    return fail("container_open: __codebook is %llu entries (quant %u), expected 2048 packed quads",
                (unsigned long long)(cb->desc.rows * cb->desc.cols), cb->desc.quant);
  std::memcpy(c->codebook, c->map + h.tensor_data_off + cb->blob_off + cb->desc.data_off, sizeof(c->codebook));
  if (!affx_codebook_valid(c->codebook))
    return fail("container_open: a __codebook byte has an E4M3 exponent outside 1..7");
  *out = c;
  return AFFX_OK;
}

void affx_container_close(affx_container* c) { close_container(c); }

uint32_t affx_container_layer_count(const affx_container* c) { return c ? (uint32_t)c->hdr->layer_count : 0u; }

int affx_container_layer(const affx_container* c, uint32_t layer, uint32_t* n_experts, uint64_t* hidden,
                         uint64_t* inter, uint64_t* stride) {
  if (!c || layer >= c->hdr->layer_count) return set_error(AFFX_ERR_ARG, "container_layer: no layer %u", layer);
  const DiskLayer& L = c->layers[layer];
  if (n_experts) *n_experts = L.n_experts;
  if (hidden) *hidden = L.gate.cols;
  if (inter) *inter = L.gate.rows;
  if (stride) *stride = L.stride;
  return AFFX_OK;
}

const void* affx_container_expert_ptr(const affx_container* c, uint32_t layer, uint32_t expert) {
  if (!c || layer >= c->hdr->layer_count || expert >= c->layers[layer].n_experts) return nullptr;
  const DiskLayer& L = c->layers[layer];
  return c->pool + L.base_off + (uint64_t)expert * L.stride;
}

int affx_container_codebook(const affx_container* c, uint32_t* out) {
  if (!c || !out) return set_error(AFFX_ERR_ARG, "container_codebook: null argument");
  std::memcpy(out, c->codebook, sizeof(c->codebook));
  return AFFX_OK;
}

int affx_container_upload_layer(const affx_container* c, uint32_t layer, void* staging, void* dst, void* stream) {
  if (!c || !staging || !dst || layer >= c->hdr->layer_count)
    return set_error(AFFX_ERR_ARG, "container_upload_layer: bad arguments");
  const DiskLayer& L = c->layers[layer];
  const uint64_t H = L.gate.cols, I = L.gate.rows;
  const uint64_t stride = affx_expert_layout(H, I, nullptr, nullptr);
  hipStream_t s = (hipStream_t)stream;
  // experts one by one at the device stride (the container's may be larger), then the permutation
  int rc = AFFX_OK;
  for (uint32_t e = 0; e < L.n_experts && !rc; ++e)
    rc = check_hip(hipMemcpyAsync((uint8_t*)staging + (uint64_t)e * stride, c->pool + L.base_off + e * L.stride,
                                  stride, hipMemcpyHostToDevice, s),
                   "container upload H2D");
  if (rc) return rc;
  return affx_permute_experts(staging, dst, L.n_experts, H, I, stream);
}

}  // extern "C"
