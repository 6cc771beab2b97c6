"""Calibration workload for HBM traffic counters: three device copies of a
256 MiB f32 buffer.  Profiling it with `rocprofv3 --pmc FETCH_SIZE` (then
WRITE_SIZE) gives the counter reading for a known number of bytes, the
scale used for the traffic figures of the decode kernel."""
import torch


def main():
    n = 256 * 1024 * 1024
    a = torch.empty(n // 4, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()


if __name__ == "__main__":
    main()
