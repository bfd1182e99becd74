/*
 * vx_host_fallback.h -- run a dispatch the GPU does not take on the host.
 *
 * A region the compiler did not classify as `kind=matmul`, and that carries no
 * device image this library can load (the compiler has no AMDGPU image
 * pipeline: reference src/dialect/VxLowering.cpp:6522-6534), runs as its
 * outlined host kernel `_vx_ciface_<name>`, called through libffi with the
 * calling convention rebuilt from the tags (reference
 * runtime/vx_host_call.h:60-130, :323-383). Operands in HBM are copied to
 * host memory for the call and back afterwards (reference
 * runtime/cuda_dispatch.cpp:1733-1860): each device view is copied as the
 * dense byte span it reaches, into a private descriptor, so the caller's
 * descriptors are never modified.
 *
 * This is the reference ABI's behaviour for unroutable regions, not a second
 * path for the routed ops: a routed GEMM that the GPU cannot run is refused
 * loudly by the dispatch library instead of landing here.
 */
#ifndef VX_AMD_HOST_FALLBACK_H
#define VX_AMD_HOST_FALLBACK_H

#include "../../include/vx_hardware_runtime.h"

#include <dlfcn.h>
#include <ffi.h>

#include <cstdint>
#include <cstring>
#include <functional>
#include <vector>

namespace vx {

inline ffi_type *ffi_type_for_tag(int32_t tag) {
  switch (VX_ABI_KIND(tag)) {
  case VX_ABI_KIND_I1:
    return &ffi_type_uint8;
  case VX_ABI_KIND_I8:
    return &ffi_type_sint8;
  case VX_ABI_KIND_I16:
    return &ffi_type_sint16;
  case VX_ABI_KIND_I32:
    return &ffi_type_sint32;
  case VX_ABI_KIND_I64:
    return &ffi_type_sint64;
  case VX_ABI_KIND_F32:
    return &ffi_type_float;
  case VX_ABI_KIND_F64:
    return &ffi_type_double;
  default:
    return &ffi_type_pointer;
  }
}

/* `_vx_ciface_<name>`, looked up first in the library holding the payload
 * (every library numbers its kernels from 0), then globally. */
inline void *host_kernel_symbol(const char *kernel_name) {
  char sym[256];
  snprintf(sym, sizeof(sym), "_vx_ciface_%s", kernel_name);
  Dl_info info;
  if (dladdr(kernel_name, &info) && info.dli_fname) {
    void *lib = dlopen(info.dli_fname, RTLD_LAZY | RTLD_NOLOAD);
    if (lib) {
      void *fn = dlsym(lib, sym);
      dlclose(lib);
      if (fn) {
        return fn;
      }
    }
  }
  return dlsym(RTLD_DEFAULT, sym);
}

/* Copy hooks: device->host and host->device of `bytes`. */
struct HostCopies {
  std::function<bool(const void *)> is_device;
  std::function<void(void *dst, const void *src, size_t bytes)> to_host;
  std::function<void(void *dst, const void *src, size_t bytes)> to_device;
};

/* One memref the call sees through a host copy. */
struct StagedView {
  std::vector<int64_t> desc; /* private descriptor storage, in 8-byte words */
  std::vector<unsigned char> bytes;
  void *device_data = nullptr; /* element [0,...] in HBM */
  size_t span = 0;
  void *desc_ptr = nullptr; /* what the argument slot points at */
  std::vector<int64_t> slot; /* for a slot argument: its own descriptor */
  void *slot_ptr = nullptr;
};

/* Descriptor words for rank r: 2 pointers + offset + 2r extents. */
inline size_t desc_words(int32_t rank) { return 3 + 2 * (size_t)rank; }

/* Build a host copy of the view `desc` if its data is in HBM; false if it is
 * not (then the argument is passed through untouched). */
inline bool stage_view(const void *desc, int32_t rank, int32_t elem,
                       const HostCopies &io, StagedView &out) {
  void *data = vx_memref_data(desc, elem);
  if (!vx_memref_aligned(desc) || !io.is_device(vx_memref_aligned(desc))) {
    return false;
  }
  uint64_t span = vx_memref_view_bytes(vx_memref_sizes(desc),
                                       vx_memref_strides(desc, rank), rank,
                                       elem);
  out.device_data = data;
  out.span = (size_t)span;
  out.bytes.resize(out.span ? out.span : 1);
  if (out.span) {
    io.to_host(out.bytes.data(), data, out.span);
  }
  out.desc.assign(desc_words(rank), 0);
  memcpy(out.desc.data(), desc, desc_words(rank) * sizeof(int64_t));
  void **ptrs = reinterpret_cast<void **>(out.desc.data());
  ptrs[0] = out.bytes.data();
  ptrs[1] = out.bytes.data();
  out.desc[2] = 0; /* offset: the copy starts at element [0,...] */
  return true;
}

/* Call `kernel` with `args`/`tags`, copying HBM views through the host.
 * Returns false when libffi rejects the signature. */
inline bool call_on_host(void *kernel, void **device_args,
                         const int32_t *arg_tags, int64_t num_args,
                         const HostCopies &io) {
  std::vector<ffi_type *> types((size_t)(num_args > 0 ? num_args : 1));
  std::vector<void *> args((size_t)(num_args > 0 ? num_args : 1));
  std::vector<StagedView> staged((size_t)(num_args > 0 ? num_args : 1));
  std::vector<bool> copied((size_t)(num_args > 0 ? num_args : 1), false);

  for (int64_t i = 0; i < num_args; ++i) {
    types[(size_t)i] = ffi_type_for_tag(arg_tags[i]);
    args[(size_t)i] = device_args[i];
    const int32_t tag = arg_tags[i];
    const int32_t rank = VX_ABI_RANK(tag);
    const int32_t elem = VX_ABI_ELEM(tag);
    if (VX_ABI_KIND(tag) != VX_ABI_KIND_MEMREF || !device_args[i] ||
        (rank == 0 && elem == VX_DTYPE_UNKNOWN) || rank > VX_ABI_MAX_RANK) {
      continue;
    }
    void *desc = *(void **)device_args[i];
    if (!desc) {
      continue;
    }
    StagedView &sv = staged[(size_t)i];
    if (VX_ABI_IS_SLOT(tag)) {
      /* A slot holds a descriptor by reference: stage the view it names and
       * point a private slot at the private descriptor. */
      void *inner = vx_memref_aligned(desc);
      if (!inner || !stage_view(inner, rank, elem, io, sv)) {
        continue;
      }
      sv.slot.assign(3, 0);
      void **sp = reinterpret_cast<void **>(sv.slot.data());
      sp[0] = sv.desc.data();
      sp[1] = sv.desc.data();
      sv.slot_ptr = sv.slot.data();
      args[(size_t)i] = &sv.slot_ptr;
    } else {
      if (!stage_view(desc, rank, elem, io, sv)) {
        continue;
      }
      sv.desc_ptr = sv.desc.data();
      args[(size_t)i] = &sv.desc_ptr;
    }
    copied[(size_t)i] = true;
  }

  ffi_cif cif;
  if (ffi_prep_cif(&cif, FFI_DEFAULT_ABI, (unsigned)num_args, &ffi_type_void,
                   types.data()) != FFI_OK) {
    return false;
  }
  ffi_call(&cif, reinterpret_cast<void (*)(void)>(kernel), nullptr,
           args.data());

  for (int64_t i = 0; i < num_args; ++i) {
    StagedView &sv = staged[(size_t)i];
    if (!copied[(size_t)i]) {
      continue;
    }
    void *now = reinterpret_cast<void **>(sv.desc.data())[1];
    if (VX_ABI_IS_SLOT(arg_tags[i]) && now != sv.bytes.data()) {
      /* The kernel published a new result through the slot: hand its
       * descriptor to the caller's storage instead of copying the old view
       * back. */
      void *inner = vx_memref_aligned(*(void **)device_args[i]);
      memcpy(inner, sv.desc.data(),
             desc_words(VX_ABI_RANK(arg_tags[i])) * sizeof(int64_t));
      continue;
    }
    if (sv.span) {
      io.to_device(sv.device_data, sv.bytes.data(), sv.span);
    }
  }
  return true;
}

} // namespace vx

#endif /* VX_AMD_HOST_FALLBACK_H */
