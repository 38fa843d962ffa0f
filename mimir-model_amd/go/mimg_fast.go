//go:build mimg

// GPU replacements for the block-quantized linear fast paths of package
// interp (reference interp/fast.go:40-59, 185-282), calling libmimg through
// its C ABI (include/mimg.h).
//
// This file belongs in the reference's interp/ directory. Build with
//
//	CGO_CFLAGS=-I<repo>/include CGO_LDFLAGS="-L<repo>/mimir-model_amd -lmimg -Wl,-rpath,<repo>/mimir-model_amd" \
//	    go build -tags mimg ./...
//
// The fastFunc signature and its callers (interp/interp.go:853-877,
// interp/plan.go:834-896) are unchanged: init() wraps the existing entries
// of fastPaths. A call the library does not handle (status > 0: a dtype or
// block without a GPU kernel, x not f32, no gfx950 GPU) runs the original Go
// function, so behaviour only changes where the GPU computes the same
// result. Set MIMG_DISABLE=1 to keep the CPU paths.
package interp

/*
#cgo LDFLAGS: -lmimg
#include "mimg.h"
*/
import "C"

import (
	"fmt"
	"os"
	"sync"
	"unsafe"

	mim "github.com/gsoultan/mimir-model"
	"github.com/gsoultan/mimir-model/ref"
)

var (
	mimgOnce sync.Once
	mimgUp   bool
)

func mimgReady() bool {
	mimgOnce.Do(func() {
		if os.Getenv("MIMG_DISABLE") == "1" {
			return
		}
		mimgUp = C.mimg_init(0) == C.MIMG_OK
	})
	return mimgUp
}

func mimgErr(op string, rc C.int) error {
	return fmt.Errorf("%s: libmimg status %d: %s", op, int(rc), C.GoString(C.mimg_last_error()))
}

// mimgWeight returns the library handle of w. The library keys its cache on
// (W.Data address, length, dtype, N, K): W.Data is a slice of the file's
// mmap, stable for the Program's life, so only the first call uploads.
func mimgWeight(w *ref.Tensor) (C.uint64_t, C.int) {
	var h C.uint64_t
	if len(w.Data) == 0 || len(w.Shape) != 2 {
		return 0, C.MIMG_NOT_HANDLED
	}
	rc := C.mimg_register_weight(unsafe.Pointer(&w.Data[0]), C.uint64_t(len(w.Data)), C.uint32_t(w.DType),
		C.int64_t(w.Shape[0]), C.int64_t(w.Shape[1]), &h)
	return h, rc
}

// mimgLinear runs y = x . W^T (+ bias) on the GPU: block > 0 is
// dequant_matmul_a8 with that activation block, block == 0 is
// dequant_matmul.v1. handled == false means "run the Go path".
func mimgLinear(in []*ref.Tensor, block int) ([]*ref.Tensor, bool, error) {
	if !mimgReady() || len(in) < 2 || len(in) > 3 {
		return nil, false, nil
	}
	if err := checkDequantMatmul(in); err != nil {
		return nil, false, err
	}
	x, w := in[0], in[1]
	switch w.DType {
	case mim.Q4_K, mim.Q6_K, mim.Q8_0:
	default:
		return nil, false, nil
	}
	k := w.Shape[1]
	if x.DType != mim.F32 || x.Shape[len(x.Shape)-1] != k {
		return nil, false, nil
	}
	var bias *C.float
	if len(in) == 3 {
		if in[2].DType != mim.F32 {
			return nil, false, nil
		}
		bias = (*C.float)(unsafe.Pointer(&f32View(in[2])[0]))
	}
	h, rc := mimgWeight(w)
	if rc != C.MIMG_OK {
		if rc > 0 {
			return nil, false, nil
		}
		return nil, false, mimgErr("register weight", rc)
	}
	rows := x.NumElems() / k
	y := make([]float32, rows*w.Shape[0])
	if rows == 0 {
		shape := append(append([]int{}, x.Shape[:len(x.Shape)-1]...), w.Shape[0])
		return []*ref.Tensor{f32Tensor(shape, y)}, true, nil
	}
	xp := (*C.float)(unsafe.Pointer(&f32View(x)[0]))
	yp := (*C.float)(unsafe.Pointer(&y[0]))
	if block > 0 {
		rc = C.mimg_dequant_matmul_a8(h, xp, C.int64_t(rows), bias, C.int(block), yp)
	} else {
		rc = C.mimg_dequant_matmul(h, xp, C.int64_t(rows), bias, yp)
	}
	if rc > 0 {
		return nil, false, nil
	}
	if rc < 0 {
		return nil, false, mimgErr("dequant_matmul", rc)
	}
	shape := append(append([]int{}, x.Shape[:len(x.Shape)-1]...), w.Shape[0])
	return []*ref.Tensor{f32Tensor(shape, y)}, true, nil
}

// withFallback runs the GPU version and, when it does not handle the call,
// the original fast path.
func withFallback(gpu, cpu fastFunc) fastFunc {
	return func(attrs []mim.Attr, in []*ref.Tensor, dts []mim.DType, shapes [][]int) ([]*ref.Tensor, bool, error) {
		out, ok, err := gpu(attrs, in, dts, shapes)
		if ok || err != nil {
			return out, ok, err
		}
		return cpu(attrs, in, dts, shapes)
	}
}

func init() {
	fastPaths["dequant_matmul.v1"] = withFallback(func(list []mim.Attr, in []*ref.Tensor, _ []mim.DType, _ [][]int) ([]*ref.Tensor, bool, error) {
		if len(list) != 0 {
			return nil, false, nil
		}
		return mimgLinear(in, 0)
	}, fastPaths["dequant_matmul.v1"])
	fastPaths["dequant_matmul_a8.v1"] = withFallback(func(list []mim.Attr, in []*ref.Tensor, _ []mim.DType, _ [][]int) ([]*ref.Tensor, bool, error) {
		if len(list) != 0 {
			return nil, false, nil
		}
		return mimgLinear(in, 32)
	}, fastPaths["dequant_matmul_a8.v1"])
	fastPaths["dequant_matmul_a8.v2"] = withFallback(func(list []mim.Attr, in []*ref.Tensor, _ []mim.DType, _ [][]int) ([]*ref.Tensor, bool, error) {
		block, err := a8Block(list)
		if err != nil {
			return nil, false, err
		}
		return mimgLinear(in, block)
	}, fastPaths["dequant_matmul_a8.v2"])
}
