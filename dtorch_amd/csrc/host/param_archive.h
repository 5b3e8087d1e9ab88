// Field-order binary archive for the operator params.
//
// The reference serialises every operator param with boost's `ar & field` idiom in a member
// `template <class Archive> void serialize(Archive&, const unsigned int)` and dispatches the type
// through its serialisation pack (dtorch/core/operators/operator_serialization_pack.h:91-140), so the
// byte layout is exactly the order of the `ar &` statements.  The params here keep that member-
// template shape (a DTorch tree instantiates it with its boost archives unchanged); this archive is
// the dependency-free instantiation used by the Python bindings (pickle) and the round-trip tests:
// little-endian fixed-width scalars, a one-byte presence flag before an optional, and a u64 length
// before a string.
#pragma once

#include <cstdint>
#include <cstring>
#include <optional>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

namespace dtorch_amd {
namespace core {

class ParamWriter {
public:
    template <typename T>
    ParamWriter& operator&(const T& v) {
        Put(v);
        return *this;
    }
    const std::string& Bytes() const { return mBuf; }

private:
    template <typename T>
    void Put(const T& v) {
        if constexpr (std::is_arithmetic_v<T>) {
            char b[sizeof(T)];
            std::memcpy(b, &v, sizeof(T));
            mBuf.append(b, sizeof(T));
        } else {
            const_cast<T&>(v).serialize(*this, 0u);
        }
    }
    void Put(const std::string& s) {
        Put(static_cast<uint64_t>(s.size()));
        mBuf.append(s);
    }
    template <typename T>
    void Put(const std::optional<T>& o) {
        Put(static_cast<uint8_t>(o.has_value() ? 1 : 0));
        if (o.has_value()) Put(*o);
    }
    std::string mBuf;
};

class ParamReader {
public:
    explicit ParamReader(std::string bytes) : mBuf(std::move(bytes)) {}
    template <typename T>
    ParamReader& operator&(T& v) {
        Get(v);
        return *this;
    }
    bool AtEnd() const { return mPos == mBuf.size(); }

private:
    template <typename T>
    void Get(T& v) {
        if constexpr (std::is_same_v<T, bool>) {
            // one byte that must be 0 or 1: any other value copied into a bool is undefined behaviour
            uint8_t byte = 0;
            Get(byte);
            if (byte > 1) throw std::invalid_argument("dtorch_amd: corrupt bool in param bytes");
            v = byte != 0;
        } else if constexpr (std::is_arithmetic_v<T>) {
            if (mBuf.size() - mPos < sizeof(T)) throw std::invalid_argument("dtorch_amd: truncated param bytes");
            std::memcpy(&v, mBuf.data() + mPos, sizeof(T));
            mPos += sizeof(T);
        } else {
            v.serialize(*this, 0u);
        }
    }
    void Get(std::string& s) {
        uint64_t n = 0;
        Get(n);
        if (mBuf.size() - mPos < n) throw std::invalid_argument("dtorch_amd: truncated param bytes");
        s.assign(mBuf.data() + mPos, n);
        mPos += n;
    }
    template <typename T>
    void Get(std::optional<T>& o) {
        uint8_t has = 0;
        Get(has);
        if (has > 1) throw std::invalid_argument("dtorch_amd: corrupt optional flag in param bytes");
        if (has) {
            T v{};
            Get(v);
            o = std::move(v);
        } else {
            o.reset();
        }
    }
    std::string mBuf;
    size_t mPos = 0;
};

// Serialise / restore a param through its serialize() member.  Restoring checks that every byte was
// consumed, so a layout mismatch fails loudly instead of yielding a half-filled param.
template <typename P>
std::string ToBytes(const P& p) {
    ParamWriter w;
    w & p;
    return w.Bytes();
}

template <typename P>
P FromBytes(const std::string& bytes) {
    P p{};
    ParamReader r(bytes);
    r & p;
    if (!r.AtEnd()) throw std::invalid_argument("dtorch_amd: trailing bytes after param");
    return p;
}

}  // namespace core
}  // namespace dtorch_amd
