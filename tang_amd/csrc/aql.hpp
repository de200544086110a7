// Recorded kernel sequences replayed on an HSA queue of the library's own
// (aql.cpp).
#pragma once

#include <functional>

#include "common.hpp"

namespace th {

// False when TANG_HIP_DISPATCH=graph (HIP graph replay instead).
bool aql_enabled();
// Record the kernels `enqueue` launches (launch_kernel) as a sequence.
// write_through: every kernel in it stores the values later kernels read with
// write-through stores, so the packets carry no fences between them.
// Anything `enqueue` puts on the stream other than a kernel is an error.
// independent (with write_through): no kernel of the sequence reads what
// another of its kernels writes, so the packets carry no acquire either.
AqlSeq* aql_record(th_device* d, bool write_through, const std::function<void()>& enqueue,
                   bool independent = false);
// Enqueue a replay, after earlier submissions (and after the device stream's
// work when nothing is in flight).  Call aql_wait before further stream work.
// repeat: the sequence `repeat` times back to back as one submission
// (system-scope fences only at its first and last packet).
void aql_submit(const AqlSeq& seq, size_t repeat = 1);
// Wait for every submitted sequence of the device.
void aql_wait(th_device* d);
void aql_free(AqlSeq* seq);
// Device clock stamps around submitted work: aql_stamp(d, 0), submissions,
// aql_stamp(d, 1), then aql_stamped_ms(d) waits and returns the interval.
void aql_stamp(th_device* d, int which);
// The stamp kernel launched on the device stream (which < 4), so that a
// sequence being recorded can carry its own stamps: aql_stamped_ms reads
// stamps 0 and 1, aql_stamp_span_ms stamps 2 and 3 (after waiting).
void aql_stamp_launch(th_device* d, int which);
float aql_stamp_span_ms(th_device* d);
float aql_stamped_ms(th_device* d);

// Device stream and AQL queue both drained.
inline void device_sync(th_device* d) {
    aql_wait(d);
    TH_HIP(hipStreamSynchronize(d->stream));
}

}  // namespace th
