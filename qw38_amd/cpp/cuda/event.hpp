// HIP events (interface of cuda/event.hpp in Enucatl/qw38).
#pragma once

#include "cuda/error.hpp"
#include "cuda/stream.hpp"

#include <hip/hip_runtime.h>

#include "qw38/expected.hpp"

namespace qw38::cuda {

class Event {
 public:
  Event() noexcept = default;
  Event(Event&& other) noexcept;
  Event& operator=(Event&& other) noexcept;
  ~Event();
  Event(Event const&) = delete;
  Event& operator=(Event const&) = delete;

  [[nodiscard]] static expected<Event, Error> create();
  [[nodiscard]] static expected<Event, Error> create_timing();
  [[nodiscard]] expected<void, Error> close();

  [[nodiscard]] hipEvent_t native() const noexcept { return event_; }
  [[nodiscard]] bool empty() const noexcept { return event_ == nullptr; }
  [[nodiscard]] int device() const noexcept { return device_; }

  [[nodiscard]] expected<void, Error> record(Stream const& stream) const;
  [[nodiscard]] expected<void, Error> wait(Stream const& stream) const;
  [[nodiscard]] expected<void, Error> sync() const;

 private:
  Event(hipEvent_t event, int device) noexcept : event_(event), device_(device) {}
  [[nodiscard]] hipError_t destroy() noexcept;
  hipEvent_t event_{nullptr};
  int device_{-1};
};

[[nodiscard]] expected<float, Error> elapsed_ms(Event const& start, Event const& end);

}  // namespace qw38::cuda
