// POSIX mmap of whole files, read-only.
#include "common/mmap_file.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <fstream>
#include <sstream>
#include <utility>

#include "common/error.hpp"

namespace ember {

MappedFile::MappedFile(const std::string &path) : path_(path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) fail("cannot open {}: {}", path, std::strerror(errno));
    struct stat st {};
    if (::fstat(fd, &st) != 0) {
        const int e = errno;
        ::close(fd);
        fail("cannot stat {}: {}", path, std::strerror(e));
    }
    size_ = static_cast<size_t>(st.st_size);
    if (size_ > 0) {
        void *p = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            const int e = errno;
            ::close(fd);
            fail("cannot map {}: {}", path, std::strerror(e));
        }
        data_ = static_cast<const uint8_t *>(p);
    }
    ::close(fd);  // the mapping keeps the file
}

MappedFile::~MappedFile() { close(); }

MappedFile::MappedFile(MappedFile &&other) noexcept
    : path_(std::move(other.path_)), data_(std::exchange(other.data_, nullptr)), size_(std::exchange(other.size_, 0)) {}

MappedFile &MappedFile::operator=(MappedFile &&other) noexcept {
    if (this != &other) {
        close();
        path_ = std::move(other.path_);
        data_ = std::exchange(other.data_, nullptr);
        size_ = std::exchange(other.size_, 0);
    }
    return *this;
}

void MappedFile::close() {
    if (data_) ::munmap(const_cast<uint8_t *>(data_), size_);
    data_ = nullptr;
    size_ = 0;
}

std::string read_file(const std::string &path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) fail("cannot read {}", path);
    std::ostringstream ss;
    ss << in.rdbuf();
    return ss.str();
}

bool file_exists(const std::string &path) {
    struct stat st {};
    return ::stat(path.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

}  // namespace ember
