// std::expected for the qw38::cuda interfaces on any C++20 toolchain.
//
// With a standard library that provides std::expected (C++23), the
// qw38::cuda names expected / unexpected / unexpect are exactly the std
// ones. Older libraries (GCC 11 libstdc++, used by hipcc in this image, also
// declares a legacy function std::unexpected) get this self-contained
// implementation in qw38::compat with the same interface subset:
// expected<T, E>, expected<void, E>, unexpected<E> with deduction,
// unexpect_t, bad_expected_access, has_value / operator bool / value /
// error / operator* / operator-> / value_or / and_then / transform_error.
#pragma once

#include <version>

#if defined(__cpp_lib_expected)
#include <expected>

namespace qw38::cuda {
using std::expected;
using std::unexpect;
using std::unexpect_t;
using std::unexpected;
}  // namespace qw38::cuda

#else

#include <exception>
#include <type_traits>
#include <utility>
#include <variant>

namespace qw38::compat {

using std::exception;
using std::enable_if_t;
using std::is_default_constructible_v;
using std::in_place_index;
using std::remove_cvref_t;
using std::invoke_result_t;
using std::variant;


template <class E>
class unexpected {
 public:
  constexpr explicit unexpected(const E& e) : e_(e) {}
  constexpr explicit unexpected(E&& e) : e_(std::move(e)) {}
  constexpr const E& error() const& noexcept { return e_; }
  constexpr E& error() & noexcept { return e_; }
  constexpr E&& error() && noexcept { return std::move(e_); }

 private:
  E e_;
};
template <class E>
unexpected(E) -> unexpected<E>;

struct unexpect_t {
  explicit unexpect_t() = default;
};
inline constexpr unexpect_t unexpect{};

template <class E>
class bad_expected_access : public exception {
 public:
  explicit bad_expected_access(E e) : e_(std::move(e)) {}
  const char* what() const noexcept override { return "bad expected access"; }
  const E& error() const& noexcept { return e_; }

 private:
  E e_;
};

template <class T, class E>
class expected {
 public:
  using value_type = T;
  using error_type = E;

  template <class U = T, class = enable_if_t<is_default_constructible_v<U>>>
  constexpr expected() : v_(in_place_index<0>) {}
  constexpr expected(const T& t) : v_(in_place_index<0>, t) {}
  constexpr expected(T&& t) : v_(in_place_index<0>, std::move(t)) {}
  template <class G>
  constexpr expected(const unexpected<G>& u) : v_(in_place_index<1>, u.error()) {}
  template <class G>
  constexpr expected(unexpected<G>&& u) : v_(in_place_index<1>, std::move(u).error()) {}
  template <class... A>
  constexpr explicit expected(unexpect_t, A&&... a) : v_(in_place_index<1>, std::forward<A>(a)...) {}

  constexpr bool has_value() const noexcept { return v_.index() == 0; }
  constexpr explicit operator bool() const noexcept { return has_value(); }

  constexpr T& value() & {
    if (!has_value()) throw bad_expected_access<E>(error());
    return std::get<0>(v_);
  }
  constexpr const T& value() const& {
    if (!has_value()) throw bad_expected_access<E>(error());
    return std::get<0>(v_);
  }
  constexpr T&& value() && {
    if (!has_value()) throw bad_expected_access<E>(error());
    return std::get<0>(std::move(v_));
  }
  constexpr T& operator*() & noexcept { return *std::get_if<0>(&v_); }
  constexpr const T& operator*() const& noexcept { return *std::get_if<0>(&v_); }
  constexpr T&& operator*() && noexcept { return std::move(*std::get_if<0>(&v_)); }
  constexpr T* operator->() noexcept { return std::get_if<0>(&v_); }
  constexpr const T* operator->() const noexcept { return std::get_if<0>(&v_); }
  constexpr E& error() & noexcept { return *std::get_if<1>(&v_); }
  constexpr const E& error() const& noexcept { return *std::get_if<1>(&v_); }
  constexpr E&& error() && noexcept { return std::move(*std::get_if<1>(&v_)); }
  template <class U>
  constexpr T value_or(U&& u) const& {
    return has_value() ? **this : static_cast<T>(std::forward<U>(u));
  }
  template <class F>
  constexpr auto and_then(F&& f) & {
    using R = remove_cvref_t<invoke_result_t<F, T&>>;
    return has_value() ? std::forward<F>(f)(**this) : R(unexpect, error());
  }
  template <class F>
  constexpr auto transform_error(F&& f) const& {
    using G = remove_cvref_t<invoke_result_t<F, const E&>>;
    return has_value() ? expected<T, G>(**this) : expected<T, G>(unexpect, std::forward<F>(f)(error()));
  }

 private:
  variant<T, E> v_;
};

template <class E>
class expected<void, E> {
 public:
  using value_type = void;
  using error_type = E;

  constexpr expected() noexcept = default;
  template <class G>
  constexpr expected(const unexpected<G>& u) : ok_(false), e_(u.error()) {}
  template <class G>
  constexpr expected(unexpected<G>&& u) : ok_(false), e_(std::move(u).error()) {}
  template <class... A>
  constexpr explicit expected(unexpect_t, A&&... a) : ok_(false), e_(std::forward<A>(a)...) {}

  constexpr bool has_value() const noexcept { return ok_; }
  constexpr explicit operator bool() const noexcept { return ok_; }
  constexpr void value() const {
    if (!ok_) throw bad_expected_access<E>(e_);
  }
  constexpr void operator*() const noexcept {}
  constexpr E& error() & noexcept { return e_; }
  constexpr const E& error() const& noexcept { return e_; }
  constexpr E&& error() && noexcept { return std::move(e_); }
  template <class F>
  constexpr auto and_then(F&& f) const& {
    using R = remove_cvref_t<invoke_result_t<F>>;
    return ok_ ? std::forward<F>(f)() : R(unexpect, e_);
  }

 private:
  bool ok_ = true;
  E e_{};
};

}  // namespace qw38::compat


namespace qw38::cuda {
using compat::expected;
using compat::unexpect;
using compat::unexpect_t;
using compat::unexpected;
}  // namespace qw38::cuda

#endif
