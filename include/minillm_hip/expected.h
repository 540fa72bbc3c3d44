// expected.h -- a minimal expected<T, E> for toolchains without C++23 <expected>.
//
// The reference host API returns std::expected<T, Status>
// (e.g. include/minillm/graph/graph_builder.h:19-35).  libstdc++ 11, the standard
// library of this image, has no <expected>, so the mirror API uses this small
// value-or-error type with the same spelling at call sites:
//   if (!r) return r.error();  use(*r);  r.value();  std::move(r).value();
//   return minillm::unexpected(Status::...);
#pragma once

#include <cassert>
#include <new>
#include <type_traits>
#include <utility>

namespace minillm {

template <typename E>
class unexpected {
 public:
  explicit unexpected(E e) : e_(std::move(e)) {}
  const E& error() const& { return e_; }
  E&& error() && { return std::move(e_); }

 private:
  E e_;
};

template <typename T, typename E>
class expected {
 public:
  expected(const T& v) : ok_(true) { new (&v_) T(v); }
  expected(T&& v) : ok_(true) { new (&v_) T(std::move(v)); }
  template <typename G>
  expected(const unexpected<G>& u) : ok_(false) { new (&e_) E(u.error()); }
  template <typename G>
  expected(unexpected<G>&& u) : ok_(false) { new (&e_) E(std::move(u).error()); }
  expected(const expected& o) : ok_(o.ok_) {
    if (ok_) new (&v_) T(o.v_); else new (&e_) E(o.e_);
  }
  expected(expected&& o) noexcept : ok_(o.ok_) {
    if (ok_) new (&v_) T(std::move(o.v_)); else new (&e_) E(std::move(o.e_));
  }
  expected& operator=(expected o) {
    this->~expected();
    new (this) expected(std::move(o));
    return *this;
  }
  ~expected() {
    if (ok_) v_.~T(); else e_.~E();
  }

  bool has_value() const { return ok_; }
  explicit operator bool() const { return ok_; }
  T& value() & { assert(ok_); return v_; }
  const T& value() const& { assert(ok_); return v_; }
  T&& value() && { assert(ok_); return std::move(v_); }
  T& operator*() & { return value(); }
  const T& operator*() const& { return value(); }
  T&& operator*() && { return std::move(v_); }
  T* operator->() { return &value(); }
  const T* operator->() const { return &value(); }
  const E& error() const& { assert(!ok_); return e_; }
  E&& error() && { assert(!ok_); return std::move(e_); }

 private:
  bool ok_;
  union {
    T v_;
    E e_;
  };
};

}  // namespace minillm
