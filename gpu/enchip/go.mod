module github.com/townsendmerino/aikit/gpu/enchip

go 1.27.0

require (
	github.com/ebitengine/purego v0.10.1
	github.com/townsendmerino/aikit v1.24.0
)

require (
	golang.org/x/sys v0.47.0 // indirect
	golang.org/x/text v0.40.0 // indirect
)

replace github.com/townsendmerino/aikit => ../../
