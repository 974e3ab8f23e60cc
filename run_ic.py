import ctypes, json, torch
lib = ctypes.CDLL("/root/repo/_work/icache/libic.so")
out = torch.zeros(1024, device="cuda")
names = ["straight_0", "straight_500", "straight_1000", "straight_2000", "straight_4000", "looped_4000"]
for w, n in enumerate(names):
    def step():
        for _ in range(28):
            assert lib.launch(w, ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
    step(); torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(3): g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(50): g.replay()
    e1.record(); torch.cuda.synchronize()
    print(json.dumps({"kernel": n, "us_per_launch": round(e0.elapsed_time(e1) * 1e3 / (50 * 28), 3)}), flush=True)
