"""Reference launches for the byte counters of rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE).

Device-to-device copies through scrapgpu_buffer_copy (the runtime's copy kernel), five launches
each of 64 MiB, 256 MiB and 1 GiB: every launch reads and writes exactly its size, so the counter
reading per launch divided by the size is the factor that turns a kernel's reading into HBM bytes
(and the three sizes show whether it depends on the size). Run under the profiler, one counter per
run:

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir> -o fetch -- python3 pmc_calibrate.py
"""
import json

import scrapgpulibrary_amd as sg

SIZES = (64 << 20, 256 << 20, 1 << 30)
LAUNCHES = 5


def main():
    dev = sg.Device(0)
    st = dev.stream()
    for n in SIZES:
        a, b = dev.alloc(n), dev.alloc(n)
        for _ in range(LAUNCHES):
            sg.check(sg.lib().scrapgpu_buffer_copy(st.handle, b.handle, 0, a.handle, 0, n, 0), "buffer_copy")
        st.sync()
        a.free()
        b.free()
    print(json.dumps({"calibration": "scrapgpu_buffer_copy", "bytes_per_launch": list(SIZES), "launches_each": LAUNCHES}))


if __name__ == "__main__":
    main()
