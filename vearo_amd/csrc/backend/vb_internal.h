// vb_internal.h -- shared by the vb_* entry points of libvearo_backend.so.
#pragma once
#include <string>

// Records msg as vb_last_error()'s text for this thread and returns code.
int vb_fail(int code, const std::string& msg);
