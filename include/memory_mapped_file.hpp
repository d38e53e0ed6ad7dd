// MemoryMappedFile: read-only mapping of a model file, with the reference's
// interface and exception texts (include/memory_mapped_file.hpp:12-95 of
// MarcVivas/llm-inference): explicit construction from a path, move-only,
// bytes() / size(), the file kept open and mapped until destruction.
#pragma once
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstddef>
#include <filesystem>
#include <span>
#include <stdexcept>
#include <system_error>

#include "model_config.hpp"

class MemoryMappedFile {
public:
    explicit MemoryMappedFile(const std::filesystem::path& path) {
        if (!std::filesystem::exists(path))
            throw std::runtime_error("File does not exist: " + path.string());
        file_size = std::filesystem::file_size(path);
        if (file_size < sizeof(ModelConfig))
            throw std::runtime_error("File is smaller than model header");
        fd = ::open(path.c_str(), O_RDONLY);
        if (fd == -1) throw std::system_error(errno, std::generic_category(), "Failed to open file");
        void* at = ::mmap(nullptr, file_size, PROT_READ, MAP_SHARED, fd, 0);
        if (at == MAP_FAILED) {
            const int e = errno;
            ::close(fd);
            fd = -1;
            throw std::system_error(e, std::generic_category(), "Failed to mmap file");
        }
        // the whole file is read once, front to back, by the upload
        ::madvise(at, file_size, MADV_WILLNEED);
        ::madvise(at, file_size, MADV_SEQUENTIAL);
        data = static_cast<const std::byte*>(at);
    }

    ~MemoryMappedFile() { reset(); }

    MemoryMappedFile(const MemoryMappedFile&) = delete;
    MemoryMappedFile& operator=(const MemoryMappedFile&) = delete;

    MemoryMappedFile(MemoryMappedFile&& o) noexcept
        : file_size(o.file_size), data(o.data), fd(o.fd) {
        o.file_size = 0;
        o.data = nullptr;
        o.fd = -1;
    }

    MemoryMappedFile& operator=(MemoryMappedFile&& o) noexcept {
        if (this != &o) {
            reset();
            file_size = o.file_size;
            data = o.data;
            fd = o.fd;
            o.file_size = 0;
            o.data = nullptr;
            o.fd = -1;
        }
        return *this;
    }

    std::span<const std::byte> bytes() const noexcept { return {data, file_size}; }
    size_t size() const noexcept { return file_size; }

private:
    size_t file_size = 0;
    const std::byte* data = nullptr;
    int fd = -1;

    void reset() noexcept {
        if (data) ::munmap(const_cast<std::byte*>(data), file_size);
        data = nullptr;
        if (fd != -1) ::close(fd);
        fd = -1;
    }
};
