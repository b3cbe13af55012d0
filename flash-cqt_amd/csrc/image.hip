// Table image check and upload, and buffer sizes (host code only).
//
// The image is the flat form of the batch-invariant tables the Python
// builder writes (flash_cqt/tables.py, image_bytes): a header, a section
// table and 256-byte aligned sections. fcqt_image_check validates every
// table against the bounds the kernels index with, on the host, before any
// HIP call; fcqt_tables_upload copies the checked image unchanged into
// caller-owned device memory, so each table's device address is the base
// plus its offset in the image.
#include <cstring>

#include "fcqt_fft.hpp"
#include "fcqt_abi_internal.hpp"

namespace fcqt {
namespace {

enum Section : uint32_t {
    kSecTwPass = 1, kSecTwHalf, kSecTwStage, kSecTasks, kSecRoute, kSecRouteB, kSecScat, kSecScatA,
    kSecOvfScat, kSecOvfScatA, kSecSliceGroups, kSecNcoef, kSecCount = kSecNcoef
};

constexpr int kRecordsPerTask = 2048;   // 16 slots x 128 threads per band task
constexpr int kImageAlign = 256;

struct SecRef {
    const uint8_t* data = nullptr;
    uint32_t elem = 0;
    uint64_t count = 0;
    uint64_t offset = 0;
};

template <typename T>
T load(const uint8_t* p) {
    T v;
    std::memcpy(&v, p, sizeof(T));
    return v;
}

int32_t i32(const SecRef& s, uint64_t i) { return load<int32_t>(s.data + 4 * i); }

bool is_band_length(int32_t M) {
    for (int m = 32; m <= 2048; m *= 2)
        if (M == m) return true;
    return false;
}

// Parse and check; on success fill secs (indexed by id) and info.
int parse(const void* image, int64_t len, SecRef* secs, fcqt_image_info* info) {
    if (!image || len < 16) return FCQT_EARG;
    const auto* b = static_cast<const uint8_t*>(image);
    if (std::memcmp(b, "FCQT", 4) != 0) return FCQT_EARG;
    const uint32_t version = load<uint32_t>(b + 4), nsec = load<uint32_t>(b + 8);
    if (version != FCQT_IMAGE_VERSION || nsec < kSecCount || nsec > 64) return FCQT_EARG;
    if ((int64_t)(16 + 24 * (uint64_t)nsec) > len) return FCQT_EARG;
    for (uint32_t k = 0; k < nsec; ++k) {
        const uint8_t* h = b + 16 + 24 * k;
        const uint32_t id = load<uint32_t>(h), elem = load<uint32_t>(h + 4);
        const uint64_t count = load<uint64_t>(h + 8), off = load<uint64_t>(h + 16);
        if (id < 1 || id > kSecCount || secs[id].data) return FCQT_EARG;      // unknown or repeated
        if (off % kImageAlign || off < 16 + 24 * (uint64_t)nsec || off > (uint64_t)len) return FCQT_EARG;
        if (elem == 0 || count > ((uint64_t)len - off) / elem) return FCQT_EARG;
        secs[id] = SecRef{b + off, elem, count, off};
    }
    for (uint32_t id = 1; id <= kSecCount; ++id)
        if (!secs[id].data) return FCQT_EARG;
    auto shape = [&](uint32_t id, uint32_t elem, uint64_t count) {
        return secs[id].elem == elem && secs[id].count == count;
    };
    // twiddles and the coefficient count
    if (!shape(kSecTwPass, 4, 2 * (uint64_t)FCQT_TW_PASS_LEN) || !shape(kSecTwHalf, 4, 2 * (uint64_t)FCQT_TW_HALF_LEN) ||
        !shape(kSecTwStage, 4, 2 * (uint64_t)FCQT_TW_STAGE_LEN) || !shape(kSecNcoef, 8, 1))
        return FCQT_EARG;
    const int64_t ncoef = load<int64_t>(secs[kSecNcoef].data);
    if (ncoef < 1 || ncoef > ((int64_t)1 << 31) / 8) return FCQT_EARG;
    // band tasks: {M, first coefficient, band count, first band}
    const SecRef& tk = secs[kSecTasks];
    if (tk.elem != 4 || tk.count < 4 || tk.count % 4 || tk.count / 4 > (1 << 20)) return FCQT_EARG;
    const int32_t ntasks = (int32_t)(tk.count / 4);
    int64_t span = 0;
    for (int32_t t = 0; t < ntasks; ++t) {
        const int32_t M = i32(tk, 4 * t), first = i32(tk, 4 * t + 1), nb = i32(tk, 4 * t + 2), band0 = i32(tk, 4 * t + 3);
        const int32_t per = M >= kRecordsPerTask ? 1 : kRecordsPerTask / M;
        if (!is_band_length(M) || nb < 1 || nb > per || first < 0 || band0 < 0) return FCQT_EARG;
        const int64_t end = (int64_t)first + (int64_t)nb * M;
        if (end > ncoef) return FCQT_EARG;
        span = end > span ? end : span;
    }
    // route records {bin, signed weight}: bins inside the spectrum
    for (uint32_t id : {kSecRoute, kSecRouteB}) {
        if (!shape(id, 4, (uint64_t)ntasks * kRecordsPerTask * 2)) return FCQT_EARG;
        for (uint64_t r = 0; r < (uint64_t)ntasks * kRecordsPerTask; ++r)
            if ((uint32_t)i32(secs[id], 2 * r) > (uint32_t)kL) return FCQT_EARG;
    }
    // scatter records {slot | mode << 30, gain}: slots inside an F row, modes 0..2
    for (uint32_t id : {kSecScat, kSecScatA}) {
        if (!shape(id, 4, (uint64_t)ntasks * kRecordsPerTask * 2)) return FCQT_EARG;
        for (uint64_t r = 0; r < (uint64_t)ntasks * kRecordsPerTask; ++r) {
            const uint32_t x = (uint32_t)i32(secs[id], 2 * r);
            if ((x & 0x3fffffffu) >= (uint32_t)kFRow || (x >> 30) > 2) return FCQT_EARG;
        }
    }
    // fold lists: -1, or bin | overflow index << 16 with bin <= L, index < cap
    for (uint32_t id : {kSecOvfScat, kSecOvfScatA}) {
        if (!shape(id, 4, FCQT_OVF_LEN)) return FCQT_EARG;
        for (uint64_t r = 0; r < FCQT_OVF_LEN; ++r) {
            const int32_t e = i32(secs[id], r);
            if (e != -1 && (e < 0 || (e & 0xffff) > kL || (e >> 16) >= kOvfCap)) return FCQT_EARG;
        }
    }
    // slice groups {first coefficient, bands, roll, 0}: each task inside its group
    const SecRef& sg = secs[kSecSliceGroups];
    if (!shape(kSecSliceGroups, 4, (uint64_t)ntasks * 4)) return FCQT_EARG;
    for (int32_t t = 0; t < ntasks; ++t) {
        const int32_t M = i32(tk, 4 * t), first = i32(tk, 4 * t + 1), nb = i32(tk, 4 * t + 2);
        const int32_t off = i32(sg, 4 * t), bins = i32(sg, 4 * t + 1), roll = i32(sg, 4 * t + 2);
        if (off < 0 || bins < 1 || (roll != 0 && roll != 1)) return FCQT_EARG;
        if ((int64_t)off + (int64_t)bins * M > ncoef || first < off || (first - off) % M) return FCQT_EARG;
        if ((int64_t)first + (int64_t)nb * M > (int64_t)off + (int64_t)bins * M) return FCQT_EARG;
    }
    if (info) {
        info->device_bytes = len;
        info->ncoef = ncoef;
        info->coef_span = span;
        info->ntasks = ntasks;
        info->format = (int32_t)version;
    }
    return FCQT_OK;
}

}  // namespace
}  // namespace fcqt

using namespace fcqt;

extern "C" int fcqt_image_check(const void* image, int64_t len, fcqt_image_info* info) {
    SecRef secs[kSecCount + 1];
    return parse(image, len, secs, info);
}

extern "C" int fcqt_tables_upload(const void* image, int64_t len, void* dev, int64_t dev_bytes, hipStream_t stream,
                                  fcqt_engine_tables* out) {
    SecRef secs[kSecCount + 1];
    fcqt_image_info info;
    if (int e = parse(image, len, secs, &info)) return e;
    if (!dev || !out || dev_bytes < info.device_bytes) return FCQT_EARG;
    if (!aligned(dev, kImageAlign)) return FCQT_EALIGN;
    hipError_t err = hipMemcpyAsync(dev, image, (size_t)len, hipMemcpyHostToDevice, stream);
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    if (err != hipSuccess) {
        std::snprintf(last_error_buf(), 256, "%s (%d)", hipGetErrorString(err), (int)err);
        return FCQT_ELAUNCH;
    }
    auto* base = static_cast<uint8_t*>(dev);
    auto at = [&](uint32_t id) { return base + secs[id].offset; };
    std::memset(out, 0, sizeof(*out));
    out->tab.tw_pass = reinterpret_cast<const float*>(at(kSecTwPass));
    out->tab.tw_half = reinterpret_cast<const float*>(at(kSecTwHalf));
    out->tab.tw_stage = reinterpret_cast<const float*>(at(kSecTwStage));
    out->tab.tasks = reinterpret_cast<const int32_t*>(at(kSecTasks));
    out->tab.ntasks = info.ntasks;
    out->tab.ncoef = info.ncoef;
    out->tab.coef_span = info.coef_span;
    out->route = reinterpret_cast<const int32_t*>(at(kSecRoute));
    out->route_b = reinterpret_cast<const int32_t*>(at(kSecRouteB));
    out->scat = reinterpret_cast<const int32_t*>(at(kSecScat));
    out->scat_a = reinterpret_cast<const int32_t*>(at(kSecScatA));
    out->ovf_scat = reinterpret_cast<const int32_t*>(at(kSecOvfScat));
    out->ovf_scat_a = reinterpret_cast<const int32_t*>(at(kSecOvfScatA));
    out->slice_groups = reinterpret_cast<const int32_t*>(at(kSecSliceGroups));
    return FCQT_OK;
}

extern "C" int fcqt_workspace_sizes(const fcqt_tables* tab, int64_t batch, fcqt_sizes* out) {
    if (!tab || !out || batch < 1 || batch > kMaxBatch || tab->ncoef < 1 || tab->ncoef > ((int64_t)1 << 31))
        return FCQT_EARG;
    out->signal = batch * (int64_t)kN * 4;
    out->spectrum = batch * (int64_t)kXStride * 8;
    out->work = batch * (int64_t)kL * 8;
    out->scatter = batch * (int64_t)kFRow * 8;
    out->coef_plane = batch * tab->ncoef * 4;
    out->tail = batch * (int64_t)(kN / 2) * 4;
    out->sync = FCQT_SYNC_WORDS(batch) * 4;
    return FCQT_OK;
}
