// MemoryMappedFile: a read-only, whole-file view of weights.bin for Model's
// constructor.  The engine builds one from a path and hands it to Model
// (src/main.cpp:19-30 of MarcVivas/llm-inference); only the class name and
// the bytes() / size() accessors are that interface.
//
// The file is mapped once, privately and read-only.  The descriptor is closed
// as soon as the mapping exists (a mapping outlives its descriptor), so the
// only resource held is the mapping itself, owned by a std::unique_ptr whose
// deleter knows the length: moves, destruction and the moved-from state come
// from unique_ptr.  Failures throw std::runtime_error naming the path, the
// system call and the errno text; a file shorter than the 44-byte header is
// rejected before anything is mapped.
#pragma once
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstddef>
#include <cstring>
#include <filesystem>
#include <memory>
#include <span>
#include <stdexcept>
#include <string>

#include "model_config.hpp"

class MemoryMappedFile {
public:
    explicit MemoryMappedFile(const std::filesystem::path& path) {
        const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd < 0) throw failure(path, "open", errno);
        struct stat st {};
        if (::fstat(fd, &st) != 0) {
            const int err = errno;
            ::close(fd);
            throw failure(path, "fstat", err);
        }
        const size_t length = static_cast<size_t>(st.st_size);
        if (length < sizeof(ModelConfig)) {
            ::close(fd);
            throw std::runtime_error(path.string() + ": " + std::to_string(length) +
                                     " bytes, shorter than the " +
                                     std::to_string(sizeof(ModelConfig)) + "-byte model header");
        }
        void* at = ::mmap(nullptr, length, PROT_READ, MAP_PRIVATE, fd, 0);
        const int err = errno;
        ::close(fd);
        if (at == MAP_FAILED) throw failure(path, "mmap", err);
        // the upload reads the payload once, front to back
        ::madvise(at, length, MADV_SEQUENTIAL);
        mapping_ = Mapping(static_cast<const std::byte*>(at), Unmap{length});
    }

    std::span<const std::byte> bytes() const noexcept { return {mapping_.get(), size()}; }
    size_t size() const noexcept { return mapping_ ? mapping_.get_deleter().length : 0; }

private:
    struct Unmap {
        size_t length = 0;
        void operator()(const std::byte* p) const noexcept {
            ::munmap(const_cast<std::byte*>(p), length);
        }
    };
    using Mapping = std::unique_ptr<const std::byte, Unmap>;
    Mapping mapping_{nullptr, Unmap{0}};

    static std::runtime_error failure(const std::filesystem::path& path, const char* call,
                                      int err) {
        return std::runtime_error(std::string(call) + "(" + path.string() +
                                  "): " + std::strerror(err));
    }
};
