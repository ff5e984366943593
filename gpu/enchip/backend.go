//go:build linux

// Package enchip is the MI355X (gfx950) encoder backend. It dlopens libenchip.so
// (a C-ABI library with embedded gfx950 code objects) with purego, so the aikit
// core stays cgo-free. Importing it registers "hip" with encoder.RegisterBackend.
package enchip

import (
	"errors"
	"fmt"
	"os"
	"runtime"
	"sync"
	"unsafe"

	"github.com/ebitengine/purego"
	"github.com/townsendmerino/aikit/ann"
	"github.com/townsendmerino/aikit/encoder"
)

func init() {
	encoder.RegisterBackend("hip", func() (encoder.Backend, error) { return New() })
	// ann takes a ready backend (ann/backend.go:139), registered only when the library
	// and a device are present, as gpu/anncuda's init does; otherwise FlatI8 keeps
	// scoring on the CPU.
	if b, err := New(); err == nil {
		ann.RegisterBackend(annBackend{b})
	}
}

// pinned runs f on one OS thread: enchip_last_error reports the failures of the calling
// thread, so a call and the read of its message must not be split across threads by the
// Go scheduler.
func pinned(f func()) {
	runtime.LockOSThread()
	defer runtime.UnlockOSThread()
	f()
}

// Status codes and activation codes of include/enchip.h.
const (
	statusOK  = 0
	actNone   = 0
	actGELU   = 1
	abiVersion = 3
)

var (
	loadOnce sync.Once
	loadErr  error

	cAbiVersion     func() int32
	cOpen           func(device int32, out *uintptr) int32
	cClose          func(ctx uintptr) int32
	cLastError      func(ctx uintptr) string
	cWeightRegister func(ctx uintptr, wq, wscale unsafe.Pointer, n, k int64, out *uint64) int32
	cWeightRelease  func(ctx uintptr, w uint64) int32
	cLinear         func(ctx uintptr, w uint64, a unsafe.Pointer, m int64, bias unsafe.Pointer,
		act int32, dst unsafe.Pointer, accDebug unsafe.Pointer) int32
	cMatmulBTF32    func(ctx uintptr, a, b, dst unsafe.Pointer, m, k, n int64) int32
	cMatmulBTQ8     func(ctx uintptr, w uint64, a unsafe.Pointer, m int64, dst unsafe.Pointer) int32
	cAnnTopK        func(ctx uintptr, w uint64, q unsafe.Pointer, m, k int64, idx, score unsafe.Pointer) int32
)

// minGPUFlops: the f32 MatmulBT dispatch threshold, enccuda's value
// (gpu/enccuda/backend.go:48-75); the device entry point itself runs any shape.
const minGPUFlops = 1 << 20

func libPath() string {
	if p := os.Getenv("AIKIT_ENCHIP_LIB"); p != "" {
		return p
	}
	return "libenchip.so"
}

func load() error {
	loadOnce.Do(func() {
		h, err := purego.Dlopen(libPath(), purego.RTLD_NOW|purego.RTLD_GLOBAL)
		if err != nil {
			loadErr = fmt.Errorf("enchip: dlopen %s: %w", libPath(), err)
			return
		}
		purego.RegisterLibFunc(&cAbiVersion, h, "enchip_abi_version")
		purego.RegisterLibFunc(&cOpen, h, "enchip_open")
		purego.RegisterLibFunc(&cClose, h, "enchip_close")
		purego.RegisterLibFunc(&cLastError, h, "enchip_last_error")
		purego.RegisterLibFunc(&cWeightRegister, h, "enchip_weight_register")
		purego.RegisterLibFunc(&cWeightRelease, h, "enchip_weight_release")
		purego.RegisterLibFunc(&cLinear, h, "enchip_w8a8_linear")
		purego.RegisterLibFunc(&cMatmulBTF32, h, "enchip_matmul_bt_f32")
		purego.RegisterLibFunc(&cMatmulBTQ8, h, "enchip_matmul_bt_q8")
		purego.RegisterLibFunc(&cAnnTopK, h, "enchip_ann_topk")
		if v := cAbiVersion(); v != abiVersion {
			loadErr = fmt.Errorf("enchip: libenchip ABI %d, binding wants %d", v, abiVersion)
		}
	})
	return loadErr
}

// Backend is the HIP encoder backend: W8A8 linears on the device, everything else
// on aikit's CPU path.
type Backend struct {
	mu  sync.Mutex // libenchip serialises host-pointer calls per context; this keeps
	ctx uintptr    // the handle map consistent too (EncodeBatch fans out goroutines)
	cpu encoder.Backend
	// Weights are write-once model parameters, so residency keyed by (ptr, len)
	// is sound (the enccuda argument, gpu/enccuda/backend.go:204-244). Activations
	// are never cached.
	weights map[wkey]uint64
}

type wkey struct {
	p uintptr
	n int
}

// New opens device 0. It fails, rather than degrading silently, when the library
// or the device is missing, so encoder.NewBackend("hip") reports the real reason.
func New() (*Backend, error) {
	if err := load(); err != nil {
		return nil, err
	}
	var ctx uintptr
	var openErr error
	pinned(func() {
		if rc := cOpen(0, &ctx); rc != statusOK {
			openErr = fmt.Errorf("enchip: open: %s (status %d)", cLastError(0), rc)
		}
	})
	if openErr != nil {
		return nil, openErr
	}
	cpu, err := encoder.NewBackend("cpu")
	if err != nil {
		cClose(ctx)
		return nil, err
	}
	return &Backend{ctx: ctx, cpu: cpu, weights: map[wkey]uint64{}}, nil
}

func (b *Backend) Name() string { return "hip" }

// MatmulBT is the f32 seam (attention's QKᵀ and scores·V, encoder/attention.go:108,111).
// a and w are uploaded on every call: attention rewrites the same pooled scratch
// between calls, so contents are never cached (gpu/enccuda/backend_test.go:88-130).
// Small shapes, and any device failure, run the CPU path (gpu/enccuda/backend.go:136-146).
func (b *Backend) MatmulBT(a, w, dst []float32, M, K, N int) {
	if 2*int64(M)*int64(K)*int64(N) < minGPUFlops || M <= 0 || K <= 0 || N <= 0 {
		b.cpu.MatmulBT(a, w, dst, M, K, N)
		return
	}
	b.mu.Lock()
	rc := cMatmulBTF32(b.ctx, unsafe.Pointer(&a[0]), unsafe.Pointer(&w[0]), unsafe.Pointer(&dst[0]),
		int64(M), int64(K), int64(N))
	b.mu.Unlock()
	if rc != statusOK {
		b.cpu.MatmulBT(a, w, dst, M, K, N)
	}
}

// MatmulBTQ8 implements encoder.Q8Backend, the weight-only int8 seam
// (encoder/backend_use.go:59-83): dst = a · (f32(wq)·wscales)ᵀ with the activations
// left in f32 (enchip_matmul_bt_q8 never quantizes them). The weight is resident per
// (ptr, len), the same registration MatmulBTW8A8 uses, and stays int8 on the device;
// a is uploaded on every call. Small shapes (enccuda's threshold,
// gpu/enccuda/backend.go:248-250) and any failure return false, and the caller runs
// matmulBTQ8Into on the CPU unchanged.
func (b *Backend) MatmulBTQ8(dst, a []float32, wq []int8, wscales []float32, M, K, N int) bool {
	if 2*int64(M)*int64(K)*int64(N) < minGPUFlops || M <= 0 || K <= 0 || N <= 0 {
		return false
	}
	if len(a) < M*K || len(wq) < N*K || len(wscales) < N || len(dst) < M*N {
		return false
	}
	b.mu.Lock()
	defer b.mu.Unlock()
	h, err := b.resident(wq[:N*K], wscales[:N], N, K)
	if err != nil {
		return false
	}
	return cMatmulBTQ8(b.ctx, h, unsafe.Pointer(&a[0]), int64(M), unsafe.Pointer(&dst[0])) == statusOK
}

// MatmulBTW8A8 implements encoder.W8A8Backend:
// dst = act(W8A8(a, wq, wscales) + bias). Returns false (decline) on any failure,
// and the caller then runs linalg's W8A8 CPU path, which gives the same bits.
func (b *Backend) MatmulBTW8A8(dst, a []float32, wq []int8, wscales, bias []float32, act, M, K, N int) bool {
	if M <= 0 || K <= 0 || N <= 0 || len(a) < M*K || len(wq) < N*K || len(wscales) < N ||
		len(dst) < M*N || (bias != nil && len(bias) < N) || (act != actNone && act != actGELU) {
		return false
	}
	b.mu.Lock()
	defer b.mu.Unlock()
	h, err := b.resident(wq[:N*K], wscales[:N], N, K)
	if err != nil {
		return false
	}
	var bp unsafe.Pointer
	if bias != nil {
		bp = unsafe.Pointer(&bias[0])
	}
	rc := cLinear(b.ctx, h, unsafe.Pointer(&a[0]), int64(M), bp, int32(act), unsafe.Pointer(&dst[0]), nil)
	return rc == statusOK
}

func (b *Backend) resident(wq []int8, ws []float32, N, K int) (uint64, error) {
	k := wkey{uintptr(unsafe.Pointer(&wq[0])), len(wq)}
	if h, ok := b.weights[k]; ok {
		return h, nil
	}
	var h uint64
	var err error
	pinned(func() {
		if rc := cWeightRegister(b.ctx, unsafe.Pointer(&wq[0]), unsafe.Pointer(&ws[0]), int64(N), int64(K), &h); rc != statusOK {
			err = errors.New(cLastError(b.ctx))
		}
	})
	if err != nil {
		return 0, err
	}
	b.weights[k] = h
	return h, nil
}

// Close frees every device buffer. The model does not own the backend
// (encoder/backend_use.go:28-29); the caller closes it.
func (b *Backend) Close() error {
	b.mu.Lock()
	defer b.mu.Unlock()
	if b.ctx != 0 {
		cClose(b.ctx)
		b.ctx = 0
	}
	return nil
}
